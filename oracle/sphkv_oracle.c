/*
 * sphkv_oracle.c -- CPU restatement of Spherical-KV's encode / page-format
 * arithmetic.  TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check and
 * bench.py's cpu_baseline leg link this as the checker.  The product never
 * calls into it.
 *
 * Every function follows a line range of the reference (paths relative to the
 * reference repository root):
 *
 *   orc_pack_bits          bitpacking.py:5-29          LSB-first bit stream
 *   orc_encode_groups      spherical_kv_pipeline.py:1130-1144
 *                          (_encode_keys_with_codebooks: norm, K/(r+EPS),
 *                           einsum 'ngi,gci->ngc', argmax)
 *   orc_radius_codes       pagebuilder.py:17-21        int8 radius codes
 *   orc_build_page         pagebuilder.py:8-33 + paging.py:20-31
 *   orc_page_bytes         spherical_kv_pipeline.py:1202-1205 (section sizes)
 *   orc_encode_append      decode_kernel.cu:10-84 (Mode-A single-token encode +
 *                          append with the running-max radius scale)
 *
 * Floating-point order.  The reference runs these ops on torch CPU in fp32.
 * Bit-exact parity needs the exact operation order torch uses, which was
 * measured against torch 2.10 CPU kernels (x86-64, MKL backend):
 *   - K_g.norm(dim=-1) over g (a multiple of 8): eight fp32 lanes, lane l
 *     accumulates fmaf(x[8s+l], x[8s+l], acc) over s, then the eight lanes are
 *     summed left to right, then sqrtf.  (ATen's vectorised last-dim norm
 *     reduction with 8-wide vectors.)
 *   - einsum 'ngi,gci->ngc' lowers to a bmm with batch G, contraction g.
 *     When N*g*C < 400 ATen uses its own naive loop: a plain fp32
 *     multiply-then-add chain over i.  Otherwise MKL sgemm (oneMKL 2024.2,
 *     AVX-512 host): for N >= 2 an fmaf chain over i = 0..g-1 starting from 0;
 *     for N = 1 (reached only by g = 16, C = 64: tier 1) MKL's M = 1 kernel,
 *     whose order was identified by exact power-of-two probes and confirmed on
 *     random data (mkl_m1_sim16 below):
 *       s01  = fmaf(d1, c1, d0*c0)
 *       L_l  = d_{l+2}*c_{l+2} + d_{l+10}*c_{l+10}   (l = 0..5, products rounded)
 *       L_6  = d8*c8,  L_7 = d9*c9 + s01
 *       M_l  = L_l + L_{l+4} (l = 0..3); (M_0 + M_2) + (M_1 + M_3)
 *   - argmax returns the first index of the maximum (strict '>').
 * Compile without -ffast-math and with -ffp-contract=off so that every
 * fmaf / '*' / '+' / '/' below is exactly one IEEE operation.
 *
 * orc_encode_append restates CUDA device code instead: nvcc (default
 * -fmad=true) contracts each `acc += a * b` and `acc += (a * b) * c` into one
 * fmaf with the last product, keeps IEEE sqrtf and '/' (-prec-sqrt,
 * -prec-div), and roundf rounds half away from zero.  Those contractions are
 * written out as fmaf below.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_EPS 1e-8f           /* config.py:5 EPS, as the fp32 scalar torch uses */
#define ORC_HEADER_BYTES 8      /* config.py:3 */

/* bitpacking.py:5-29: bit j of value i lands at global bit i*bits + j. */
void orc_pack_bits(const int32_t* vals, int64_t n, int bits, uint8_t* out)
{
    int64_t total_bytes = (n * bits + 7) / 8;
    memset(out, 0, (size_t)total_bytes);
    for (int64_t i = 0; i < n; ++i) {
        for (int j = 0; j < bits; ++j) {
            if ((vals[i] >> j) & 1) {
                int64_t gb = i * bits + j;
                out[gb >> 3] = (uint8_t)(out[gb >> 3] + (1u << (gb & 7)));
            }
        }
    }
}

/* Inverse of orc_pack_bits (used to check round trips). */
void orc_unpack_bits(const uint8_t* in, int64_t n, int bits, int32_t* vals)
{
    for (int64_t i = 0; i < n; ++i) {
        int32_t v = 0;
        for (int j = 0; j < bits; ++j) {
            int64_t gb = i * bits + j;
            v |= ((in[gb >> 3] >> (gb & 7)) & 1) << j;
        }
        vals[i] = v;
    }
}

/* torch CPU fp32 L2 norm of one contiguous group of g (g % 8 == 0). */
static float torch_norm_f32(const float* x, int g)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int d = 0;
    for (; d + 8 <= g; d += 8)
        for (int l = 0; l < 8; ++l)
            acc[l] = fmaf(x[d + l], x[d + l], acc[l]);
    float b = acc[0];
    for (int l = 1; l < 8; ++l) b = b + acc[l];
    for (; d < g; ++d) b = b + x[d] * x[d];
    return sqrtf(b);
}

/* MKL's M = 1 sgemm order for a contraction of 16 (see the header). */
static float mkl_m1_sim16(const float* d, const float* c)
{
    float L[8];
    const float s01 = fmaf(d[1], c[1], d[0] * c[0]);
    for (int l = 0; l < 6; ++l) L[l] = d[l + 2] * c[l + 2] + d[l + 10] * c[l + 10];
    L[6] = d[8] * c[8];
    L[7] = d[9] * c[9] + s01;
    float M[4];
    for (int l = 0; l < 4; ++l) M[l] = L[l] + L[l + 4];
    return (M[0] + M[2]) + (M[1] + M[3]);
}

/*
 * spherical_kv_pipeline.py:1130-1144.
 * K: [N, G*g] fp32 row-major; cb: [G, C, g] fp32 (unit rows).
 * r_out: [N, G]; code_out: [N, G] int32.  Returns 0.
 */
int orc_encode_groups(const float* K, int64_t N, int G, int g,
                      const float* cb, int C, float* r_out, int32_t* code_out)
{
    const int naive = (N * (int64_t)g * C) < 400;
    const int m1 = !naive && N == 1 && g == 16;
    float dir[64];
    for (int64_t n = 0; n < N; ++n) {
        for (int gi = 0; gi < G; ++gi) {
            const float* x = K + n * (int64_t)G * g + (int64_t)gi * g;
            float r = torch_norm_f32(x, g);
            float den = r + ORC_EPS;
            for (int i = 0; i < g; ++i) dir[i] = x[i] / den;
            const float* cbg = cb + (int64_t)gi * C * g;
            int best = 0;
            float best_sim = 0.f;
            for (int c = 0; c < C; ++c) {
                float s = 0.f;
                if (naive) {
                    for (int i = 0; i < g; ++i) { float p = dir[i] * cbg[c * g + i]; s = s + p; }
                } else if (m1) {
                    s = mkl_m1_sim16(dir, cbg + c * g);
                } else {
                    for (int i = 0; i < g; ++i) s = fmaf(dir[i], cbg[c * g + i], s);
                }
                if (c == 0 || s > best_sim) { best_sim = s; best = c; }
            }
            r_out[n * G + gi] = r;
            code_out[n * G + gi] = best;
        }
    }
    return 0;
}

/* pagebuilder.py:17-21.  r: [N, G] -> scale [G], codes int8 [N, G]. */
void orc_radius_codes(const float* r, int N, int G, float* scale_out, int8_t* codes_out)
{
    for (int gi = 0; gi < G; ++gi) {
        float m = 0.f;
        for (int n = 0; n < N; ++n) {
            float a = fabsf(r[n * G + gi]);
            if (n == 0 || a > m) m = a;
        }
        scale_out[gi] = m;
    }
    for (int gi = 0; gi < G; ++gi) {
        float safe = scale_out[gi] < 1e-8f ? 1e-8f : scale_out[gi];
        for (int n = 0; n < N; ++n) {
            float q = r[n * G + gi] / safe;
            q = q * 127.0f;
            q = nearbyintf(q);                       /* torch.round: half to even */
            if (q > 127.f) q = 127.f;
            if (q < -127.f) q = -127.f;
            codes_out[n * G + gi] = (int8_t)q;
        }
    }
}

/* Section sizes of one packed page (spherical_kv_pipeline.py:1202-1205). */
int64_t orc_page_bytes(int N, int G, int b_theta)
{
    return ORC_HEADER_BYTES + 4 * (int64_t)G + ((int64_t)N * G * b_theta + 7) / 8 + (int64_t)N * G;
}

/*
 * pagebuilder.py:8-33 + paging.py:20-31.  Writes header | packed theta |
 * int8 radius into out; returns the page size in bytes.
 */
int64_t orc_build_page(const float* r, const int32_t* codes, int N, int G,
                       int b_theta, int tier_id, uint8_t* out)
{
    float scale[64];
    int8_t rc[16 * 1024];
    int32_t masked[16 * 1024];
    if (G > 64 || (int64_t)N * G > 16 * 1024) return -1;
    orc_radius_codes(r, N, G, scale, rc);
    memset(out, 0, ORC_HEADER_BYTES);
    out[0] = (uint8_t)(tier_id & 0xFF);
    out[1] = (uint8_t)(N & 0xFF);
    memcpy(out + ORC_HEADER_BYTES, scale, 4 * (size_t)G);   /* little-endian fp32 */
    uint8_t* th = out + ORC_HEADER_BYTES + 4 * G;
    for (int i = 0; i < N * G; ++i) masked[i] = codes[i];
    orc_pack_bits(masked, (int64_t)N * G, b_theta, th);
    int64_t tb = ((int64_t)N * G * b_theta + 7) / 8;
    memcpy(th + tb, rc, (size_t)N * G);
    return ORC_HEADER_BYTES + 4 * (int64_t)G + tb + (int64_t)N * G;
}

/*
 * decode_kernel.cu:10-84 for one kv head h.  Pools: theta / radius uint8
 * [n_pages, page_size, G_max], r_scales fp32 [n_pages, G_max], v_pool fp16
 * bits (uint16) [n_pages, page_size, dh].  k, v fp32 [dh]; cb fp32 [G, C, g]
 * (this head's decode codebook).  v is rounded to fp16 by the caller (the
 * kernel writes __float2half, round to nearest even).
 */
void orc_encode_append(const float* k, const float* cb, uint8_t* theta, uint8_t* radius, float* r_scales,
                       int64_t pid, int slot, int G, int g, int C, int G_max, int page_size, int is_new_page)
{
    const int64_t code_base = (pid * page_size + slot) * G_max;
    for (int grp = 0; grp < G; ++grp) {
        const float* kg = k + grp * g;
        float norm_sq = 0.f;
        for (int d = 0; d < g; ++d) norm_sq = fmaf(kg[d], kg[d], norm_sq);          /* :38-40 */
        const float norm = sqrtf(norm_sq + 1e-16f);                                 /* :41 */
        const float inv_norm = 1.0f / (norm + 1e-8f);                               /* :42 */
        const float* cbg = cb + (int64_t)grp * C * g;
        float best_sim = -1e30f;
        int best_code = 0;
        for (int c = 0; c < C; ++c) {                                               /* :45-55 */
            float sim = 0.f;
            for (int d = 0; d < g; ++d) sim = fmaf(kg[d] * inv_norm, cbg[c * g + d], sim);
            if (sim > best_sim) { best_sim = sim; best_code = c; }
        }
        theta[code_base + grp] = (uint8_t)best_code;                               /* :57 */
        float r_scale;                                                              /* :59-79 */
        if (is_new_page) {
            r_scales[pid * G_max + grp] = norm;
            r_scale = norm;
        } else {
            const float prev = r_scales[pid * G_max + grp];
            if (norm > prev) {
                const float ratio = prev / (norm + 1e-8f);
                for (int t = 0; t < slot; ++t) {
                    uint8_t* rc = radius + (pid * page_size + t) * G_max + grp;
                    float x = (float)(*rc) * ratio;
                    x = fminf(fmaxf(roundf(x), 0.f), 255.f);
                    *rc = (uint8_t)x;
                }
                r_scales[pid * G_max + grp] = norm;
                r_scale = norm;
            } else {
                r_scale = prev;
            }
        }
        float r_q = roundf(norm / (r_scale + 1e-8f) * 255.0f);                      /* :80-82 */
        r_q = fminf(fmaxf(r_q, 0.f), 255.f);
        radius[code_base + grp] = (uint8_t)r_q;
    }
}
