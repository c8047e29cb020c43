/*
 * numeric_tables.c - exhaustive and sampled checks of the element
 * conversions and libm restatements the gfx950 kernels compile from
 * (m3.c_amd/csrc/hip/m3_numeric.h, m3_libm.h), built for the host.
 *
 * TEST INFRASTRUCTURE. Modes:
 *   numeric_tables tables <impl> [<library>]
 *       Prints the hashes of the four full conversion tables of one
 *       implementation: F32->F16 and F32->BF16 over all 2^32 F32 bit
 *       patterns, F16->F32 and BF16->F32 over all 2^16 patterns.
 *       impl = product   the kernels' header, compiled here;
 *              planted   the product with one F32->F16 entry (input
 *                        0x3f800fff) rounded the wrong way, to show that
 *                        the hash detects a single wrong entry;
 *              oracle    the oracle restatement (oracle/liboracle.so);
 *              reference the reference's own CAST on its CPU provider
 *                        (oracle/_ref/libm3ref.so, src/m3_op_execute_basic.c
 *                        :28-59 through src/m3_op_numeric.c:27-130).
 *   numeric_tables compare <oracle library>
 *       Compares the product and oracle conversions value by value over
 *       the same domains and prints the number of differences.
 *   numeric_tables libm <stride>
 *       Compares m3_expf and m3_sinf with the C library's expf and sinf
 *       on every stride-th float (expf on floats <= 0.5, the softmax
 *       domain; sinf on all floats), the magnitude of
 *       m3_sinf_medium_magnitude with that of sinf where |x| < 120, and
 *       m3_expf_any, m3_expm1f, m3_tanhf and m3_tanhf_uniform with expf,
 *       expm1f and tanhf on the same floats and on the edges of
 *       m3_tanhf_common's domain (m3_tanhf_common there too), and m3_gated_silu_bits (F32 gate)
 *       and m3_silu_quotient_fast (its quotient alone, NaN as a class)
 *       with the same statements in C on every stride-th gate, each with
 *       one of eight non-NaN up values (the product then has at most one
 *       NaN operand, so its NaN bits are fixed by IEEE 754 and x86-64),
 *       and prints the mismatch counts.
 *   numeric_tables silu16
 *       m3_gated_silu_bits for F16 and BF16 gates: every 16-bit gate with
 *       each of the eight up values, against the C statements with the
 *       activation rounded through the gate's dtype by the converters.
 *
 * Table hash: the inputs are split into blocks of 2^16 consecutive bit
 * patterns; each block's outputs (little-endian, 2 or 4 bytes each) are
 * hashed with 64-bit FNV-1a, and the block hashes (8 bytes each, in block
 * order) are hashed again with FNV-1a.
 */
#include "m3_activation.h"
#include "m3_libm.h"
#include "m3_numeric.h"

#include <dlfcn.h>
#include <inttypes.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define FNV_OFFSET 0xcbf29ce484222325ULL
#define FNV_PRIME 0x100000001b3ULL
#define BLOCK (1U << 16)

static uint64_t fnv_bytes(uint64_t h, const uint8_t *p, size_t n)
{
    for (size_t i = 0U; i < n; ++i) {
        h ^= p[i];
        h *= FNV_PRIME;
    }
    return h;
}

typedef uint16_t (*narrow_fn)(uint32_t bits);
typedef uint32_t (*widen_fn)(uint16_t half);

/* ---- product (the kernels' header) ---- */
static uint16_t product_f32_f16(uint32_t b)
{
    return (uint16_t)m3_f32_to_f16_bits(b);
}

static uint16_t product_f32_bf16(uint32_t b)
{
    return (uint16_t)m3_f32_to_bf16_bits(b);
}

static uint32_t product_f16_f32(uint16_t h)
{
    return m3_f16_to_f32_bits(h);
}

static uint32_t product_bf16_f32(uint16_t h)
{
    return m3_bf16_to_f32_bits(h);
}

static uint16_t planted_f32_f16(uint32_t b)
{
    uint16_t r = product_f32_f16(b);

    return b == 0x3f800fffU ? (uint16_t)(r + 1U) : r;
}

/* ---- oracle (dlopen'd) ---- */
static uint16_t (*oracle_f32_f16)(uint32_t);
static uint16_t (*oracle_f32_bf16)(uint32_t);
static uint32_t (*oracle_f16_f32)(uint16_t);
static uint32_t (*oracle_bf16_f32)(uint16_t);

static void *open_or_die(const char *path)
{
    void *handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);

    if (handle == NULL) {
        fprintf(stderr, "cannot load %s: %s\n", path, dlerror());
        exit(2);
    }
    return handle;
}

static void *symbol_or_die(void *handle, const char *name)
{
    void *p = dlsym(handle, name);

    if (p == NULL) {
        fprintf(stderr, "missing symbol %s\n", name);
        exit(2);
    }
    return p;
}

static void load_oracle(const char *path)
{
    void *h = open_or_die(path);

    *(void **)&oracle_f32_f16 = symbol_or_die(h, "oracle_f32_to_f16");
    *(void **)&oracle_f32_bf16 = symbol_or_die(h, "oracle_f32_to_bf16");
    *(void **)&oracle_f16_f32 = symbol_or_die(h, "oracle_f16_to_f32");
    *(void **)&oracle_bf16_f32 = symbol_or_die(h, "oracle_bf16_to_f32");
}

/* ---- reference (ref_execute of oracle/ref_driver.c, CAST) ---- */
typedef struct {
    void *data;
    size_t bytes;
    uint64_t byte_offset;
    uint32_t dtype;
    uint32_t rank;
    uint64_t shape[8];
    uint64_t byte_strides[8];
} ref_view;

static int (*ref_execute)(int, const ref_view *, size_t, char *, size_t);

enum { OP_CAST = 1, DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

/* The reference's CAST of `count` elements of in_dtype into out_dtype. */
static void ref_cast(const void *in, uint32_t in_dtype, void *out,
                     uint32_t out_dtype, size_t count)
{
    ref_view views[2];
    char message[256];
    size_t in_size = in_dtype == DT_F32 ? 4U : 2U;
    size_t out_size = out_dtype == DT_F32 ? 4U : 2U;

    memset(views, 0, sizeof(views));
    views[0].data = (void *)in;
    views[0].bytes = count * in_size;
    views[0].dtype = in_dtype;
    views[0].rank = 1U;
    views[0].shape[0] = count;
    views[0].byte_strides[0] = in_size;
    views[1].data = out;
    views[1].bytes = count * out_size;
    views[1].dtype = out_dtype;
    views[1].rank = 1U;
    views[1].shape[0] = count;
    views[1].byte_strides[0] = out_size;
    if (ref_execute(OP_CAST, views, 2U, message, sizeof(message)) != 0) {
        fprintf(stderr, "reference cast failed: %s\n", message);
        exit(3);
    }
}

/* Hash of the F32 -> 16-bit table over all 2^32 inputs. */
static uint64_t narrow_table_hash(narrow_fn f, uint32_t ref_dtype)
{
    const size_t blocks = (size_t)1 << 16;
    uint64_t *block_hash = malloc(blocks * sizeof(uint64_t));
    uint64_t h = FNV_OFFSET;

    if (block_hash == NULL) {
        exit(4);
    }
#pragma omp parallel
    {
        uint32_t *in = malloc(BLOCK * sizeof(uint32_t));
        uint16_t *out = malloc(BLOCK * sizeof(uint16_t));

#pragma omp for schedule(dynamic, 64)
        for (size_t b = 0; b < blocks; ++b) {
            for (uint32_t i = 0U; i < BLOCK; ++i) {
                in[i] = (uint32_t)(b * BLOCK + i);
            }
            if (f != NULL) {
                for (uint32_t i = 0U; i < BLOCK; ++i) {
                    out[i] = f(in[i]);
                }
            } else {
                ref_cast(in, DT_F32, out, ref_dtype, BLOCK);
            }
            block_hash[b] = fnv_bytes(FNV_OFFSET, (const uint8_t *)out,
                                      BLOCK * sizeof(uint16_t));
        }
        free(in);
        free(out);
    }
    for (size_t b = 0; b < blocks; ++b) {
        h = fnv_bytes(h, (const uint8_t *)&block_hash[b], 8U);
    }
    free(block_hash);
    return h;
}

/* Hash of the 16-bit -> F32 table over all 2^16 inputs (one block). */
static uint64_t widen_table_hash(widen_fn f, uint32_t ref_dtype)
{
    uint16_t in[BLOCK];
    static uint32_t out[BLOCK];
    uint64_t block;

    for (uint32_t i = 0U; i < BLOCK; ++i) {
        in[i] = (uint16_t)i;
    }
    if (f != NULL) {
        for (uint32_t i = 0U; i < BLOCK; ++i) {
            out[i] = f(in[i]);
        }
    } else {
        ref_cast(in, ref_dtype, out, DT_F32, BLOCK);
    }
    block = fnv_bytes(FNV_OFFSET, (const uint8_t *)out, sizeof(out));
    return fnv_bytes(FNV_OFFSET, (const uint8_t *)&block, 8U);
}

static int tables(const char *impl, const char *library)
{
    narrow_fn f16 = NULL;
    narrow_fn bf16 = NULL;
    widen_fn from_f16 = NULL;
    widen_fn from_bf16 = NULL;

    if (strcmp(impl, "product") == 0 || strcmp(impl, "planted") == 0) {
        f16 = strcmp(impl, "planted") == 0 ? planted_f32_f16
                                           : product_f32_f16;
        bf16 = product_f32_bf16;
        from_f16 = product_f16_f32;
        from_bf16 = product_bf16_f32;
    } else if (strcmp(impl, "oracle") == 0 && library != NULL) {
        load_oracle(library);
        f16 = oracle_f32_f16;
        bf16 = oracle_f32_bf16;
        from_f16 = oracle_f16_f32;
        from_bf16 = oracle_bf16_f32;
    } else if (strcmp(impl, "reference") == 0 && library != NULL) {
        *(void **)&ref_execute =
            symbol_or_die(open_or_die(library), "ref_execute");
    } else {
        fprintf(stderr, "unknown implementation or missing library\n");
        return 2;
    }
    printf("{\"f32_to_f16\": \"%016" PRIx64 "\", ",
           narrow_table_hash(f16, DT_F16));
    printf("\"f32_to_bf16\": \"%016" PRIx64 "\", ",
           narrow_table_hash(bf16, DT_BF16));
    printf("\"f16_to_f32\": \"%016" PRIx64 "\", ",
           widen_table_hash(from_f16, DT_F16));
    printf("\"bf16_to_f32\": \"%016" PRIx64 "\"}\n",
           widen_table_hash(from_bf16, DT_BF16));
    return 0;
}

static int compare(const char *library)
{
    unsigned long long bad = 0ULL;

    load_oracle(library);
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t u = 0; u <= (int64_t)0xffffffffLL; ++u) {
        uint32_t b = (uint32_t)u;

        bad += product_f32_f16(b) != oracle_f32_f16(b);
        bad += product_f32_bf16(b) != oracle_f32_bf16(b);
    }
    for (uint32_t h = 0U; h < BLOCK; ++h) {
        bad += product_f16_f32((uint16_t)h) != oracle_f16_f32((uint16_t)h);
        bad += product_bf16_f32((uint16_t)h) != oracle_bf16_f32((uint16_t)h);
    }
    printf("{\"conversion_mismatches\": %llu}\n", bad);
    return bad == 0ULL ? 0 : 1;
}

/* Up values of the GATED_SILU checks: signs, zero, infinities, overflow,
 * a subnormal. */
static const float silu_ups[8] = {1.0F, -0.75F, 0.0F, INFINITY, -INFINITY,
                                  3.0e38F, 1.0e-40F, 2.5F};

/* F16 and BF16 gates: all 2^16 gate patterns with each up value. */
static int silu16(void)
{
    unsigned long long checked = 0ULL;
    unsigned long long bad = 0ULL;
    uint32_t dtype;

    for (dtype = M3N_F16; dtype <= M3N_BF16; ++dtype) {
        uint32_t raw;

        for (raw = 0U; raw < 65536U; ++raw) {
            float gate = m3_bits_f32(m3_load_as_f32_bits(raw, dtype));
            int k;

            for (k = 0; k < 8; ++k) {
                volatile float denominator = 1.0F + expf(-gate);
                volatile float quotient = gate / denominator;
                float activation = m3_bits_f32(m3_round_through_bits(
                    m3_f32_bits(quotient), dtype));
                volatile float product = activation * silu_ups[k];
                float want = product;
                uint32_t got = m3_gated_silu_bits(gate, silu_ups[k], dtype);

                checked += 1U;
                bad += memcmp(&got, &want, sizeof(got)) != 0;
            }
        }
    }
    printf("{\"silu16_checked\": %llu, \"silu16_mismatches\": %llu}\n",
           checked, bad);
    return bad == 0ULL ? 0 : 1;
}

static int libm(uint64_t stride)
{
    unsigned long long exp_checked = 0ULL;
    unsigned long long exp_bad = 0ULL;
    unsigned long long sin_checked = 0ULL;
    unsigned long long sin_bad = 0ULL;
    unsigned long long magnitude_checked = 0ULL;
    unsigned long long magnitude_bad = 0ULL;
    unsigned long long other_checked = 0ULL;
    unsigned long long expf_any_bad = 0ULL;
    unsigned long long expm1f_bad = 0ULL;
    unsigned long long tanhf_bad = 0ULL;
    unsigned long long tanhf_uniform_bad = 0ULL;
    unsigned long long silu_bad = 0ULL;
    unsigned long long silu_fast_bad = 0ULL;

#pragma omp parallel for reduction(+ : exp_checked, exp_bad, sin_checked, \
                                       sin_bad, magnitude_checked,         \
                                       magnitude_bad, other_checked,       \
                                       expf_any_bad, expm1f_bad,           \
                                       tanhf_bad, tanhf_uniform_bad,       \
                                       silu_bad, silu_fast_bad)            \
    schedule(static)
    for (int64_t u = 0; u <= (int64_t)0xffffffffLL; u += (int64_t)stride) {
        uint32_t b = (uint32_t)u;
        float x;

        memcpy(&x, &b, sizeof(x));
        if (!isnan(x) && x <= 0.5F) {
            float got = m3_expf(x);
            float want = expf(x);

            exp_checked += 1U;
            exp_bad += memcmp(&got, &want, sizeof(got)) != 0;
        }
        {
            float got = m3_sinf(x);
            float want = sinf(x);

            sin_checked += 1U;
            sin_bad += memcmp(&got, &want, sizeof(got)) != 0;
            if (fabsf(x) < 120.0F) {
                float magnitude = fabsf(m3_sinf_medium_magnitude(x));

                want = fabsf(want);
                magnitude_checked += 1U;
                magnitude_bad +=
                    memcmp(&magnitude, &want, sizeof(magnitude)) != 0;
            }
        }
        {
            float got = m3_expf_any(x);
            float want = expf(x);

            other_checked += 1U;
            expf_any_bad += memcmp(&got, &want, sizeof(got)) != 0;
            got = m3_expm1f(x);
            want = expm1f(x);
            expm1f_bad += memcmp(&got, &want, sizeof(got)) != 0;
            got = m3_tanhf(x);
            want = tanhf(x);
            tanhf_bad += memcmp(&got, &want, sizeof(got)) != 0;
            got = m3_tanhf_uniform(x);
            tanhf_uniform_bad += memcmp(&got, &want, sizeof(got)) != 0;
        }
        {
            float up = silu_ups[(b >> 5) & 7U];
            volatile float denominator = 1.0F + expf(-x);
            volatile float activation = x / denominator;
            volatile float product = activation * up;
            float want = product;
            uint32_t got = m3_gated_silu_bits(x, up, M3N_F32);

            silu_bad += memcmp(&got, &want, sizeof(got)) != 0;
            {
                float quotient = activation;
                float fast = m3_silu_quotient_fast(x, m3_expf_table);

                silu_fast_bad += isnan(quotient)
                                     ? !isnan(fast)
                                     : memcmp(&fast, &quotient,
                                              sizeof(fast)) != 0;
            }
        }
    }
    /* the edges of m3_tanhf_common's domain and of its choice of k (each
     * with both signs and its neighbours): 2^-55, the first |x| with
     * k >= 23, 1 (the two expm1f arguments), the one argument where the
     * rounded k is -1 and expm1f's own is 0 (|x| = 0x1.62e43p-3), the end
     * of expm1f's k = -1 range (|x| = 1.5 ln2 / 2), and 22 */
    {
        static const uint32_t edges[] = {0x24000000U, 0x40f98872U,
                                         0x3f800000U, 0x3e317218U,
                                         0x3e317219U, 0x3f051592U,
                                         0x41b00000U};
        unsigned e;

        for (e = 0U; e < sizeof(edges) / sizeof(edges[0]); ++e) {
            uint32_t d;

            for (d = 0U; d < 6U; ++d) {
                uint32_t b = (edges[e] + d - 2U) | ((d & 1U) << 31U);
                float x;
                float got;
                float want;

                memcpy(&x, &b, sizeof(x));
                got = m3_tanhf_uniform(x);
                want = tanhf(x);
                other_checked += 1U;
                tanhf_uniform_bad += memcmp(&got, &want, sizeof(got)) != 0;
                if ((b & 0x7fffffffU) >= 0x24000000U &&
                    (b & 0x7fffffffU) < 0x40f98872U) {
                    got = m3_tanhf_common(x);
                    tanhf_uniform_bad +=
                        memcmp(&got, &want, sizeof(got)) != 0;
                }
            }
        }
    }
    printf("{\"expf_checked\": %llu, \"expf_mismatches\": %llu, "
           "\"sinf_checked\": %llu, \"sinf_mismatches\": %llu, "
           "\"sinf_magnitude_checked\": %llu, "
           "\"sinf_magnitude_mismatches\": %llu, \"all_checked\": %llu, "
           "\"expf_any_mismatches\": %llu, \"expm1f_mismatches\": %llu, "
           "\"tanhf_mismatches\": %llu, "
           "\"tanhf_uniform_mismatches\": %llu, "
           "\"gated_silu_mismatches\": %llu, "
           "\"silu_fast_mismatches\": %llu}\n",
           exp_checked, exp_bad, sin_checked, sin_bad, magnitude_checked,
           magnitude_bad, other_checked, expf_any_bad, expm1f_bad, tanhf_bad,
           tanhf_uniform_bad, silu_bad, silu_fast_bad);
    return exp_bad == 0ULL && sin_bad == 0ULL && magnitude_bad == 0ULL &&
                   expf_any_bad == 0ULL && expm1f_bad == 0ULL &&
                   tanhf_bad == 0ULL && tanhf_uniform_bad == 0ULL &&
                   silu_bad == 0ULL && silu_fast_bad == 0ULL
               ? 0
               : 1;
}

int main(int argc, char **argv)
{
    if (argc >= 3 && strcmp(argv[1], "tables") == 0) {
        return tables(argv[2], argc >= 4 ? argv[3] : NULL);
    }
    if (argc == 3 && strcmp(argv[1], "compare") == 0) {
        return compare(argv[2]);
    }
    if (argc == 3 && strcmp(argv[1], "libm") == 0) {
        return libm(strtoull(argv[2], NULL, 10));
    }
    if (argc == 2 && strcmp(argv[1], "silu16") == 0) {
        return silu16();
    }
    fprintf(stderr, "usage: numeric_tables tables|compare|libm|silu16 ...\n");
    return 2;
}
