/*
 * TEST INFRASTRUCTURE ONLY -- the CPU baseline, never the product.
 *
 * A C restatement of the path inference.rs's CPU QMatMul takes on x86-64
 * (crates/inference-tensor/src/quantized/repack_x86.rs, repack.rs:219-262,
 * avx.rs): weights re-tiled as 16 rows x one 256-value superblock with the
 * sub-block scales pre-multiplied into f32, activations quantized to Q8_K
 * (K-quants) or to per-superblock Q8_0 groups (Q8_0), and integer dots by
 * vpdpbusd (AVX-512 VNNI, or AVX-VNNI / AVX2 on 256-bit lanes), with AMX
 * tdpbssd for Q4_K at m >= 32.  The instruction level is chosen at run time
 * as repack_x86::level() does.  Shapes the tiles do not take run
 * k_quants::matmul with avx.rs's AVX2 vec_dot (Q6_K at m = 1, Q8_0 at m = 1
 * on AVX2-only CPUs), or the scalar oracle where the reference itself has no
 * x86 kernel.
 *
 * bench.py times it as the reference's CPU QMatMul beside the GPU; tests
 * check it against the scalar oracle (oracle.c) and float64 brute force.
 * Every function is compiled for a generic x86-64 target and enables its
 * instruction set with a target attribute, as the reference's
 * #[target_feature] functions do, so one build runs on any host and picks
 * its path at run time.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <immintrin.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/syscall.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define TILE_N 16
#define MAX_MT 4

/* ------------------------------------------------------------------ tiles (repack_x86.rs:12-47) */

/* one superblock of 16 rows: f32 d*sc and dmin*m per sub-block and row; nibbles as [k8-group][row][4 bytes],
 * byte j of group g holding value 8g + j (low nibble) and 8g + j + 4 (high nibble) */
typedef struct { float scales[8][TILE_N]; float mins[8][TILE_N]; uint8_t qs[32 * TILE_N * 4]; } x86_tile_q4k;
/* d*scale per 16-value sub-block; raw 6-bit values (0..63) as [k4-group][row][4 bytes] */
typedef struct { float scales[16][TILE_N]; uint8_t qs[64 * TILE_N * 4]; } x86_tile_q6k;
/* one 32-value block of 16 rows, values + 128 as [k4-group][row][4 bytes] */
typedef struct { uint16_t d[TILE_N]; uint8_t qs[32 * TILE_N]; } x86_tile_q8_0;
/* AMX form of a Q4_K superblock: unsigned 4-bit values as bytes, [sub-block][k4-row][16 cols x 4 k]
 * (repack_x86.rs:930-938) */
typedef struct { float scales[8][TILE_N]; float mins[8][TILE_N]; uint8_t qs[256 * TILE_N]; } x86_tile_q4k_amx;

/* one superblock of Q8_0 activations: eight blocks' f32 scales, integer sums and values (repack_x86.rs:53-85) */
typedef struct { float d[8]; int32_t sums[8]; int8_t qs[256]; } x86_act_q8_0;

/* ------------------------------------------------------------------ instruction level (repack_x86.rs:1305-1342) */

enum { X86_NONE = 0, X86_AVX2 = 1, X86_AVXVNNI = 2, X86_AVX512VNNI = 3 };

static int env_is_one(const char *name) {
    const char *v = getenv(name);
    return v && strcmp(v, "1") == 0;
}

/* repack_x86::level: AVX-512 F + VNNI, else AVX-VNNI (+AVX2), else AVX2 + FMA; the reference's two environment
 * switches force the lower levels */
int oracle_x86_level(void) {
    __builtin_cpu_init();
    int force_avx2 = env_is_one("MISTRALRS_FORCE_AVX2"), force_vnni = env_is_one("MISTRALRS_FORCE_AVXVNNI");
    if (!force_avx2 && !force_vnni && __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vnni"))
        return X86_AVX512VNNI;
    if (!force_avx2 && (force_vnni || __builtin_cpu_supports("avxvnni")) && __builtin_cpu_supports("avx2"))
        return X86_AVXVNNI;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return X86_AVX2;
    return X86_NONE;
}

/* repack_x86::amx_available (repack_x86.rs:985-1024): AVX-512 VNNI level, CPUID.7.0:EDX bits 24 (AMX-TILE) and
 * 25 (AMX-INT8), and Linux's per-process permission for the tile data state (arch_prctl ARCH_REQ_XCOMP_PERM) */
int oracle_x86_amx(void) {
    static int cached = -1; /* the CPUID and permission part; the level is read on every call (tests force it) */
    if (oracle_x86_level() != X86_AVX512VNNI) return 0;
    if (cached < 0) {
        unsigned a, b, c, d;
        __asm__ volatile("cpuid" : "=a"(a), "=b"(b), "=c"(c), "=d"(d) : "a"(7), "c"(0));
        int ok = 0;
        if ((d & (1u << 25)) && (d & (1u << 24)))
            ok = syscall(SYS_arch_prctl, 0x1023 /* ARCH_REQ_XCOMP_PERM */, 18 /* XFEATURE_XTILEDATA */) == 0;
        cached = ok;
    }
    return cached;
}

/* repack_x86::select (repack_x86.rs:100-121) */
int oracle_x86_select(int type, int64_t m, int64_t n, int64_t k) {
    int lv = oracle_x86_level();
    if (lv == X86_NONE) return 0;
    int64_t block = (type == OR_Q8_0) ? OR_QK8_0 : OR_QK_K;
    if (k == 0 || n % TILE_N || k % block) return 0;
    switch (type) {
    case OR_Q4K: return 1;
    case OR_Q6K: return m > 1;
    case OR_Q8_0: return lv != X86_AVX2 || m > 1;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ packing (repack_x86.rs:181-300, 1026-1066) */

static void get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static void q4k_values(const or_block_q4k *blk, uint8_t vals[256]) {
    for (int c = 0; c < 4; c++)
        for (int j = 0; j < 32; j++) {
            vals[c * 64 + j] = blk->qs[c * 32 + j] & 0x0F;
            vals[c * 64 + 32 + j] = blk->qs[c * 32 + j] >> 4;
        }
}

static void q4k_scales(const or_block_q4k *blk, float scales[8][TILE_N], float mins[8][TILE_N], int r) {
    float d = oracle_f16_to_f32(blk->d), dmin = oracle_f16_to_f32(blk->dmin);
    for (int sub = 0; sub < 8; sub++) {
        uint8_t sc, mn;
        get_scale_min_k4(sub, blk->scales, &sc, &mn);
        scales[sub][r] = d * (float)sc;
        mins[sub][r] = dmin * (float)mn;
    }
}

static void pack_q4k(const or_block_q4k *blocks, int64_t n, int64_t kb, x86_tile_q4k *out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n / TILE_N; t++)
        for (int64_t b = 0; b < kb; b++) {
            x86_tile_q4k *tile = &out[t * kb + b];
            for (int r = 0; r < TILE_N; r++) {
                const or_block_q4k *blk = &blocks[(t * TILE_N + r) * kb + b];
                uint8_t vals[256];
                q4k_scales(blk, tile->scales, tile->mins, r);
                q4k_values(blk, vals);
                for (int g = 0; g < 32; g++)
                    for (int j = 0; j < 4; j++)
                        tile->qs[(g * TILE_N + r) * 4 + j] = (uint8_t)(vals[g * 8 + j] | (vals[g * 8 + j + 4] << 4));
            }
        }
}

static void pack_q4k_amx(const or_block_q4k *blocks, int64_t n, int64_t kb, x86_tile_q4k_amx *out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n / TILE_N; t++)
        for (int64_t b = 0; b < kb; b++) {
            x86_tile_q4k_amx *tile = &out[t * kb + b];
            for (int r = 0; r < TILE_N; r++) {
                const or_block_q4k *blk = &blocks[(t * TILE_N + r) * kb + b];
                uint8_t vals[256];
                q4k_scales(blk, tile->scales, tile->mins, r);
                q4k_values(blk, vals);
                for (int sub = 0; sub < 8; sub++)
                    for (int krow = 0; krow < 8; krow++)
                        for (int j = 0; j < 4; j++)
                            tile->qs[((sub * 8 + krow) * TILE_N + r) * 4 + j] = vals[sub * 32 + krow * 4 + j];
            }
        }
}

static void pack_q6k(const or_block_q6k *blocks, int64_t n, int64_t kb, x86_tile_q6k *out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n / TILE_N; t++)
        for (int64_t b = 0; b < kb; b++) {
            x86_tile_q6k *tile = &out[t * kb + b];
            for (int r = 0; r < TILE_N; r++) {
                const or_block_q6k *blk = &blocks[(t * TILE_N + r) * kb + b];
                float d = oracle_f16_to_f32(blk->d);
                for (int sub = 0; sub < 16; sub++) tile->scales[sub][r] = d * (float)blk->scales[sub];
                uint8_t vals[256];
                for (int h = 0; h < 2; h++) {
                    const uint8_t *ql = blk->ql + h * 64, *qh = blk->qh + h * 32;
                    for (int j = 0; j < 32; j++) {
                        vals[h * 128 + j] = (uint8_t)((ql[j] & 0x0F) | ((qh[j] & 3) << 4));
                        vals[h * 128 + j + 32] = (uint8_t)((ql[j + 32] & 0x0F) | (((qh[j] >> 2) & 3) << 4));
                        vals[h * 128 + j + 64] = (uint8_t)((ql[j] >> 4) | (((qh[j] >> 4) & 3) << 4));
                        vals[h * 128 + j + 96] = (uint8_t)((ql[j + 32] >> 4) | (((qh[j] >> 6) & 3) << 4));
                    }
                }
                for (int g = 0; g < 64; g++)
                    for (int j = 0; j < 4; j++) tile->qs[(g * TILE_N + r) * 4 + j] = vals[g * 4 + j];
            }
        }
}

/* Q8_0: kb superblocks of eight blocks per row; blocks past the row end get a zero scale and +128 values
 * (a zero weight) */
static void pack_q8_0(const or_block_q8_0 *blocks, int64_t n, int64_t k, x86_tile_q8_0 *out) {
    int64_t row_blocks = k / OR_QK8_0, kb8 = (k + OR_QK_K - 1) / OR_QK_K * 8;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n / TILE_N; t++)
        for (int64_t b = 0; b < kb8; b++) {
            x86_tile_q8_0 *tile = &out[t * kb8 + b];
            memset(tile->d, 0, sizeof tile->d);
            if (b >= row_blocks) {
                memset(tile->qs, 128, sizeof tile->qs);
                continue;
            }
            for (int r = 0; r < TILE_N; r++) {
                const or_block_q8_0 *blk = &blocks[(t * TILE_N + r) * row_blocks + b];
                tile->d[r] = blk->d;
                for (int g = 0; g < 8; g++)
                    for (int j = 0; j < 4; j++)
                        tile->qs[(g * TILE_N + r) * 4 + j] = (uint8_t)((int)blk->qs[g * 4 + j] + 128);
            }
        }
}

/* a prepared weight: its blocks and the tile forms the reference caches beside them (repack.rs:35-70) */
typedef struct {
    int type;
    int64_t n, k, kb;
    const void *blocks;
    void *tiles;     /* x86_tile_q4k / _q6k / _q8_0, or NULL when select() never takes this shape */
    void *amx_tiles; /* x86_tile_q4k_amx for Q4_K when AMX is available */
} x86_weight;

/* Packs the weight as the reference's PackedCache would hold it after its first calls.  `blocks` must outlive
 * the handle.  Returns NULL on a type the x86 kernels do not serve. */
void *oracle_x86_prepare(int type, const void *blocks, int64_t n, int64_t k) {
    if (type != OR_Q4K && type != OR_Q6K && type != OR_Q8_0) return NULL;
    x86_weight *w = calloc(1, sizeof *w);
    if (!w) return NULL;
    w->type = type;
    w->n = n;
    w->k = k;
    w->kb = (k + OR_QK_K - 1) / OR_QK_K;
    w->blocks = blocks;
    /* m = 2 asks whether any batch takes the tiles (Q6_K's only at m > 1; Q8_0's at m = 1 unless AVX2-only) */
    if (oracle_x86_select(type, 2, n, k)) {
        size_t tiles = (size_t)(n / TILE_N) * (size_t)w->kb;
        size_t bytes = type == OR_Q4K ? tiles * sizeof(x86_tile_q4k)
                     : type == OR_Q6K ? tiles * sizeof(x86_tile_q6k) : tiles * 8 * sizeof(x86_tile_q8_0);
        if (posix_memalign(&w->tiles, 64, bytes)) { free(w); return NULL; }
        if (type == OR_Q4K) pack_q4k(blocks, n, w->kb, w->tiles);
        else if (type == OR_Q6K) pack_q6k(blocks, n, w->kb, w->tiles);
        else pack_q8_0(blocks, n, k, w->tiles);
        if (type == OR_Q4K && oracle_x86_amx()) {
            if (posix_memalign(&w->amx_tiles, 64, tiles * sizeof(x86_tile_q4k_amx))) {
                free(w->tiles);
                free(w);
                return NULL;
            }
            pack_q4k_amx(blocks, n, w->kb, w->amx_tiles);
        }
    }
    return w;
}

void oracle_x86_release(void *handle) {
    x86_weight *w = handle;
    if (!w) return;
    free(w->tiles);
    free(w->amx_tiles);
    free(w);
}

/* ------------------------------------------------------------------ worker pool (utils.rs:323-387, 538-581) */

/* the threads the reference runs on by default: physical cores (candle_num_threads without overrides), counted
 * here over the CPUs this process may run on */
int oracle_x86_physical_cores(void) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof set, &set) != 0) return 1;
    int seen[4096], nseen = 0;
    for (int cpu = 0; cpu < CPU_SETSIZE; cpu++) {
        if (!CPU_ISSET(cpu, &set)) continue;
        char path[128];
        int pkg = 0, core = cpu;
        snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/core_id", cpu);
        FILE *f = fopen(path, "r");
        if (f) { if (fscanf(f, "%d", &core) != 1) core = cpu; fclose(f); }
        snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/physical_package_id", cpu);
        f = fopen(path, "r");
        if (f) { if (fscanf(f, "%d", &pkg) != 1) pkg = 0; fclose(f); }
        int key = pkg * 65536 + core, dup = 0;
        for (int i = 0; i < nseen; i++) dup |= seen[i] == key;
        if (!dup && nseen < 4096) seen[nseen++] = key;
    }
    return nseen > 0 ? nseen : 1;
}

typedef void (*x86_range_fn)(void *ctx, int64_t begin, int64_t end);

/* BarrierPool::execute_chunked / execute_static: the threads pull ranges of `chunk` items from a shared cursor;
 * chunked ranges are about an eighth of a thread's share, static ranges a whole share */
static void run_ranges(int threads, int64_t items, int static_ranges, x86_range_fn fn, void *ctx) {
    if (items <= 0) return;
    int64_t chunk = static_ranges ? (items + threads - 1) / threads : (items + (int64_t)threads * 8 - 1) / ((int64_t)threads * 8);
    if (chunk < 1) chunk = 1;
    _Atomic int64_t cursor = 0;
#pragma omp parallel num_threads(threads)
    {
        for (;;) {
            int64_t start = atomic_fetch_add_explicit(&cursor, chunk, memory_order_relaxed);
            if (start >= items) break;
            fn(ctx, start, start + chunk < items ? start + chunk : items);
        }
    }
}

/* ------------------------------------------------------------------ activations (repack_x86.rs:866-912) */

/* ActQ8_0::quantize_row: quantize_block32 per 32 values with the f16 scale, read back as f32, and each block's
 * integer sum */
static void act_q8_0_row(const float *row, int64_t kb, x86_act_q8_0 *out) {
    for (int64_t b = 0; b < kb; b++) {
        or_block_q8_0 blk[8];
        oracle_quantize_q8_0(row + b * OR_QK_K, OR_QK_K, blk);
        for (int j = 0; j < 8; j++) {
            out[b].d[j] = oracle_f16_to_f32(blk[j].d);
            int32_t s = 0;
            for (int i = 0; i < 32; i++) s += blk[j].qs[i];
            out[b].sums[j] = s;
            memcpy(out[b].qs + j * 32, blk[j].qs, 32);
        }
    }
}

typedef struct { const float *lhs; int64_t k, kb; void *out; int q8_0; } quant_ctx;

/* quantize_rows: a row short of whole superblocks is quantized from a zero-padded copy */
static void quant_rows(void *vctx, int64_t begin, int64_t end) {
    quant_ctx *c = vctx;
    float *pad = NULL;
    if (c->k != c->kb * OR_QK_K) pad = calloc((size_t)(c->kb * OR_QK_K), sizeof(float));
    for (int64_t r = begin; r < end; r++) {
        const float *row = c->lhs + r * c->k;
        if (pad) { memcpy(pad, row, (size_t)c->k * sizeof(float)); row = pad; }
        if (c->q8_0) act_q8_0_row(row, c->kb, (x86_act_q8_0 *)c->out + r * c->kb);
        else oracle_quantize_q8k(row, c->kb * OR_QK_K, (or_block_q8k *)c->out + r * c->kb);
    }
    free(pad);
}

/* ------------------------------------------------------------------ AVX-512 VNNI kernels (repack_x86.rs:493-650) */

#define T512 __attribute__((target("avx512f,avx512bw,avx512vnni,fma,f16c")))

T512 static inline __m512i bcast4_512(const int8_t *p) {
    int32_t v;
    memcpy(&v, p, 4);
    return _mm512_set1_epi32(v);
}

/* q4k_tile: sub-blocks in pairs with independent integer accumulators; the min term through the Q8_K bsums */
T512 static void q4k_tile_512(const x86_tile_q4k *tile, const or_block_q8k *const *acts, int mt, __m512 *acc) {
    const __m512i mask = _mm512_set1_epi8(0x0F);
    for (int sub2 = 0; sub2 < 4; sub2++) {
        int sa = sub2 * 2, sb = sa + 1;
        __m512i isa[MAX_MT], isb[MAX_MT];
        for (int m = 0; m < mt; m++) isa[m] = isb[m] = _mm512_setzero_si512();
        for (int g4 = 0; g4 < 4; g4++) {
            __m512i wa = _mm512_loadu_si512(tile->qs + (sa * 4 + g4) * TILE_N * 4);
            __m512i wb = _mm512_loadu_si512(tile->qs + (sb * 4 + g4) * TILE_N * 4);
            __m512i lo_a = _mm512_and_si512(wa, mask), hi_a = _mm512_and_si512(_mm512_srli_epi16(wa, 4), mask);
            __m512i lo_b = _mm512_and_si512(wb, mask), hi_b = _mm512_and_si512(_mm512_srli_epi16(wb, 4), mask);
            for (int m = 0; m < mt; m++) {
                const int8_t *q = acts[m]->qs;
                isa[m] = _mm512_dpbusd_epi32(isa[m], lo_a, bcast4_512(q + sa * 32 + g4 * 8));
                isa[m] = _mm512_dpbusd_epi32(isa[m], hi_a, bcast4_512(q + sa * 32 + g4 * 8 + 4));
                isb[m] = _mm512_dpbusd_epi32(isb[m], lo_b, bcast4_512(q + sb * 32 + g4 * 8));
                isb[m] = _mm512_dpbusd_epi32(isb[m], hi_b, bcast4_512(q + sb * 32 + g4 * 8 + 4));
            }
        }
        for (int h = 0; h < 2; h++) {
            int sub = h ? sb : sa;
            __m512i *is = h ? isb : isa;
            __m512 scale = _mm512_loadu_ps(tile->scales[sub]), min = _mm512_loadu_ps(tile->mins[sub]);
            for (int m = 0; m < mt; m++) {
                float dall = acts[m]->d;
                acc[m] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(is[m]), _mm512_mul_ps(scale, _mm512_set1_ps(dall)), acc[m]);
                float bsum = (float)((int32_t)acts[m]->bsums[sub * 2] + (int32_t)acts[m]->bsums[sub * 2 + 1]);
                acc[m] = _mm512_fnmadd_ps(min, _mm512_set1_ps(dall * bsum), acc[m]);
            }
        }
    }
}

/* q6k_tile: dpbusd on the raw unsigned 6-bit values, then 32 * bsum off per 16-value sub-block */
T512 static void q6k_tile_512(const x86_tile_q6k *tile, const or_block_q8k *const *acts, int mt, __m512 *acc) {
    for (int sub = 0; sub < 16; sub++) {
        __m512i is[MAX_MT];
        for (int m = 0; m < mt; m++) is[m] = _mm512_setzero_si512();
        for (int g4 = 0; g4 < 4; g4++) {
            __m512i w = _mm512_loadu_si512(tile->qs + (sub * 4 + g4) * TILE_N * 4);
            for (int m = 0; m < mt; m++)
                is[m] = _mm512_dpbusd_epi32(is[m], w, bcast4_512(acts[m]->qs + sub * 16 + g4 * 4));
        }
        __m512 scale = _mm512_loadu_ps(tile->scales[sub]);
        for (int m = 0; m < mt; m++) {
            float dall = acts[m]->d, bsum = (float)acts[m]->bsums[sub];
            __m512 f = _mm512_sub_ps(_mm512_cvtepi32_ps(is[m]), _mm512_set1_ps(32.0f * bsum));
            acc[m] = _mm512_fmadd_ps(f, _mm512_mul_ps(scale, _mm512_set1_ps(dall)), acc[m]);
        }
    }
}

/* q8_0_tile2: two 32-value blocks with independent accumulators; the +128 offset comes off through the sums */
T512 static void q8_0_tile2_512(const x86_tile_q8_0 *t0, const x86_tile_q8_0 *t1, const x86_act_q8_0 *const *acts,
                                int mt, int sub32, __m512 *acc) {
    __m512i ia[MAX_MT], ib[MAX_MT];
    for (int m = 0; m < mt; m++) ia[m] = ib[m] = _mm512_setzero_si512();
    for (int g4 = 0; g4 < 8; g4++) {
        __m512i wa = _mm512_loadu_si512(t0->qs + g4 * TILE_N * 4), wb = _mm512_loadu_si512(t1->qs + g4 * TILE_N * 4);
        for (int m = 0; m < mt; m++) {
            ia[m] = _mm512_dpbusd_epi32(ia[m], wa, bcast4_512(acts[m]->qs + sub32 * 32 + g4 * 4));
            ib[m] = _mm512_dpbusd_epi32(ib[m], wb, bcast4_512(acts[m]->qs + (sub32 + 1) * 32 + g4 * 4));
        }
    }
    for (int h = 0; h < 2; h++) {
        const x86_tile_q8_0 *t = h ? t1 : t0;
        int blk = sub32 + h;
        __m512i *is = h ? ib : ia;
        __m512 dw = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)t->d));
        for (int m = 0; m < mt; m++) {
            __m512 f = _mm512_sub_ps(_mm512_cvtepi32_ps(is[m]), _mm512_set1_ps(128.0f * (float)acts[m]->sums[blk]));
            acc[m] = _mm512_fmadd_ps(f, _mm512_mul_ps(dw, _mm512_set1_ps(acts[m]->d[blk])), acc[m]);
        }
    }
}

typedef struct { const x86_weight *w; const void *lhs_q; int64_t m; float *dst; int level; } tiles_ctx;

/* matmul_unit_512: one 16-column tile against up to MAX_MT activation rows over the whole K range */
T512 static void unit_512(const tiles_ctx *c, int64_t nt, int64_t m0, int mt) {
    const x86_weight *w = c->w;
    int64_t kb = w->kb;
    __m512 acc[MAX_MT];
    for (int i = 0; i < MAX_MT; i++) acc[i] = _mm512_setzero_ps();
    for (int64_t b = 0; b < kb; b++) {
        if (w->type == OR_Q8_0) {
            const x86_act_q8_0 *acts[MAX_MT];
            for (int i = 0; i < mt; i++) acts[i] = (const x86_act_q8_0 *)c->lhs_q + (m0 + i) * kb + b;
            const x86_tile_q8_0 *t = (const x86_tile_q8_0 *)w->tiles + nt * kb * 8 + b * 8;
            for (int s = 0; s < 8; s += 2) q8_0_tile2_512(t + s, t + s + 1, acts, mt, s, acc);
        } else {
            const or_block_q8k *acts[MAX_MT];
            for (int i = 0; i < mt; i++) acts[i] = (const or_block_q8k *)c->lhs_q + (m0 + i) * kb + b;
            if (w->type == OR_Q4K) q4k_tile_512((const x86_tile_q4k *)w->tiles + nt * kb + b, acts, mt, acc);
            else q6k_tile_512((const x86_tile_q6k *)w->tiles + nt * kb + b, acts, mt, acc);
        }
    }
    for (int i = 0; i < mt; i++) _mm512_storeu_ps(c->dst + (m0 + i) * w->n + nt * TILE_N, acc[i]);
}

/* ------------------------------------------------------------------ 256-bit kernels (repack_x86.rs:1344-1648) */

#define T256 __attribute__((target("avx2,fma,f16c")))
#define T256V __attribute__((target("avx2,fma,f16c,avxvnni")))

T256 static inline __m256i bcast4_256(const int8_t *p) {
    int32_t v;
    memcpy(&v, p, 4);
    return _mm256_set1_epi32(v);
}

/* dpbusd stand-in for plain AVX2: maddubs (u8 x i8 -> i16 pairs), then madd against ones */
T256 static inline __m256i dp_avx2(__m256i acc, __m256i w, __m256i a) {
    return _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_maddubs_epi16(w, a), _mm256_set1_epi16(1)));
}
T256V static inline __m256i dp_vnni(__m256i acc, __m256i w, __m256i a) { return _mm256_dpbusd_avx_epi32(acc, w, a); }

/* one body per instruction level, as the reference's q4k_tile_256! / q6k_tile_256! macros */
#define Q4K_TILE_256(NAME, ATTR, DP)                                                                            \
    ATTR static void NAME(const x86_tile_q4k *tile, const or_block_q8k *const *acts, int mt, __m256 acc[][2]) { \
        const __m256i mask = _mm256_set1_epi8(0x0F);                                                            \
        for (int sub = 0; sub < 8; sub++) {                                                                     \
            __m256i is[MAX_MT][2];                                                                              \
            for (int m = 0; m < mt; m++) is[m][0] = is[m][1] = _mm256_setzero_si256();                          \
            for (int g4 = 0; g4 < 4; g4++)                                                                      \
                for (int h = 0; h < 2; h++) {                                                                   \
                    __m256i w = _mm256_loadu_si256((const __m256i *)(tile->qs + (sub * 4 + g4) * TILE_N * 4 + h * 32)); \
                    __m256i lo = _mm256_and_si256(w, mask), hi = _mm256_and_si256(_mm256_srli_epi16(w, 4), mask); \
                    for (int m = 0; m < mt; m++) {                                                              \
                        is[m][h] = DP(is[m][h], lo, bcast4_256(acts[m]->qs + sub * 32 + g4 * 8));               \
                        is[m][h] = DP(is[m][h], hi, bcast4_256(acts[m]->qs + sub * 32 + g4 * 8 + 4));           \
                    }                                                                                           \
                }                                                                                               \
            for (int h = 0; h < 2; h++) {                                                                       \
                __m256 scale = _mm256_loadu_ps(tile->scales[sub] + h * 8), min = _mm256_loadu_ps(tile->mins[sub] + h * 8); \
                for (int m = 0; m < mt; m++) {                                                                  \
                    float dall = acts[m]->d;                                                                    \
                    acc[m][h] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(is[m][h]), _mm256_mul_ps(scale, _mm256_set1_ps(dall)), acc[m][h]); \
                    float bsum = (float)((int32_t)acts[m]->bsums[sub * 2] + (int32_t)acts[m]->bsums[sub * 2 + 1]); \
                    acc[m][h] = _mm256_fnmadd_ps(min, _mm256_set1_ps(dall * bsum), acc[m][h]);                  \
                }                                                                                               \
            }                                                                                                   \
        }                                                                                                       \
    }
Q4K_TILE_256(q4k_tile_avx2, T256, dp_avx2)
Q4K_TILE_256(q4k_tile_avxvnni, T256V, dp_vnni)

#define Q6K_TILE_256(NAME, ATTR, DP)                                                                            \
    ATTR static void NAME(const x86_tile_q6k *tile, const or_block_q8k *const *acts, int mt, __m256 acc[][2]) { \
        for (int sub = 0; sub < 16; sub++) {                                                                    \
            __m256i is[MAX_MT][2];                                                                              \
            for (int m = 0; m < mt; m++) is[m][0] = is[m][1] = _mm256_setzero_si256();                          \
            for (int g4 = 0; g4 < 4; g4++)                                                                      \
                for (int h = 0; h < 2; h++) {                                                                   \
                    __m256i w = _mm256_loadu_si256((const __m256i *)(tile->qs + (sub * 4 + g4) * TILE_N * 4 + h * 32)); \
                    for (int m = 0; m < mt; m++)                                                                \
                        is[m][h] = DP(is[m][h], w, bcast4_256(acts[m]->qs + sub * 16 + g4 * 4));                \
                }                                                                                               \
            for (int h = 0; h < 2; h++) {                                                                       \
                __m256 scale = _mm256_loadu_ps(tile->scales[sub] + h * 8);                                      \
                for (int m = 0; m < mt; m++) {                                                                  \
                    float dall = acts[m]->d, bsum = (float)acts[m]->bsums[sub];                                 \
                    __m256 f = _mm256_sub_ps(_mm256_cvtepi32_ps(is[m][h]), _mm256_set1_ps(32.0f * bsum));       \
                    acc[m][h] = _mm256_fmadd_ps(f, _mm256_mul_ps(scale, _mm256_set1_ps(dall)), acc[m][h]);      \
                }                                                                                               \
            }                                                                                                   \
        }                                                                                                       \
    }
Q6K_TILE_256(q6k_tile_avx2, T256, dp_avx2)
Q6K_TILE_256(q6k_tile_avxvnni, T256V, dp_vnni)

/* q8_0_tile2_avx2: the +128 weights would saturate maddubs' i16 pairs, so |w| takes the unsigned side and w's
 * sign moves onto the activation (no offset correction) */
T256 static void q8_0_tile2_avx2(const x86_tile_q8_0 *t0, const x86_tile_q8_0 *t1, const x86_act_q8_0 *const *acts,
                                 int mt, int sub32, __m256 acc[][2]) {
    const __m256i offset = _mm256_set1_epi8((char)0x80), ones = _mm256_set1_epi16(1);
    __m256i ia[MAX_MT][2], ib[MAX_MT][2];
    for (int m = 0; m < mt; m++) ia[m][0] = ia[m][1] = ib[m][0] = ib[m][1] = _mm256_setzero_si256();
    for (int g4 = 0; g4 < 8; g4++)
        for (int h = 0; h < 2; h++) {
            __m256i wa = _mm256_xor_si256(_mm256_loadu_si256((const __m256i *)(t0->qs + g4 * TILE_N * 4 + h * 32)), offset);
            __m256i wb = _mm256_xor_si256(_mm256_loadu_si256((const __m256i *)(t1->qs + g4 * TILE_N * 4 + h * 32)), offset);
            __m256i abs_a = _mm256_sign_epi8(wa, wa), abs_b = _mm256_sign_epi8(wb, wb);
            for (int m = 0; m < mt; m++) {
                __m256i xa = _mm256_sign_epi8(bcast4_256(acts[m]->qs + sub32 * 32 + g4 * 4), wa);
                __m256i xb = _mm256_sign_epi8(bcast4_256(acts[m]->qs + (sub32 + 1) * 32 + g4 * 4), wb);
                ia[m][h] = _mm256_add_epi32(ia[m][h], _mm256_madd_epi16(_mm256_maddubs_epi16(abs_a, xa), ones));
                ib[m][h] = _mm256_add_epi32(ib[m][h], _mm256_madd_epi16(_mm256_maddubs_epi16(abs_b, xb), ones));
            }
        }
    for (int s = 0; s < 2; s++) {
        const x86_tile_q8_0 *t = s ? t1 : t0;
        int blk = sub32 + s;
        for (int h = 0; h < 2; h++) {
            __m256 dw = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(t->d + h * 8)));
            for (int m = 0; m < mt; m++) {
                __m256i is = s ? ib[m][h] : ia[m][h];
                acc[m][h] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(is), _mm256_mul_ps(dw, _mm256_set1_ps(acts[m]->d[blk])), acc[m][h]);
            }
        }
    }
}

/* q8_0_tile2_avxvnni: dpbusd takes the +128 weights as they are; the offset comes off through the sums */
T256V static void q8_0_tile2_avxvnni(const x86_tile_q8_0 *t0, const x86_tile_q8_0 *t1,
                                     const x86_act_q8_0 *const *acts, int mt, int sub32, __m256 acc[][2]) {
    __m256i ia[MAX_MT][2], ib[MAX_MT][2];
    for (int m = 0; m < mt; m++) ia[m][0] = ia[m][1] = ib[m][0] = ib[m][1] = _mm256_setzero_si256();
    for (int g4 = 0; g4 < 8; g4++)
        for (int h = 0; h < 2; h++) {
            __m256i wa = _mm256_loadu_si256((const __m256i *)(t0->qs + g4 * TILE_N * 4 + h * 32));
            __m256i wb = _mm256_loadu_si256((const __m256i *)(t1->qs + g4 * TILE_N * 4 + h * 32));
            for (int m = 0; m < mt; m++) {
                ia[m][h] = _mm256_dpbusd_avx_epi32(ia[m][h], wa, bcast4_256(acts[m]->qs + sub32 * 32 + g4 * 4));
                ib[m][h] = _mm256_dpbusd_avx_epi32(ib[m][h], wb, bcast4_256(acts[m]->qs + (sub32 + 1) * 32 + g4 * 4));
            }
        }
    for (int s = 0; s < 2; s++) {
        const x86_tile_q8_0 *t = s ? t1 : t0;
        int blk = sub32 + s;
        for (int h = 0; h < 2; h++) {
            __m256 dw = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(t->d + h * 8)));
            for (int m = 0; m < mt; m++) {
                __m256i is = s ? ib[m][h] : ia[m][h];
                __m256 f = _mm256_sub_ps(_mm256_cvtepi32_ps(is), _mm256_set1_ps(128.0f * (float)acts[m]->sums[blk]));
                acc[m][h] = _mm256_fmadd_ps(f, _mm256_mul_ps(dw, _mm256_set1_ps(acts[m]->d[blk])), acc[m][h]);
            }
        }
    }
}

/* matmul_unit_256 */
#define UNIT_256(NAME, ATTR, Q4K, Q6K, Q80)                                                                     \
    ATTR static void NAME(const tiles_ctx *c, int64_t nt, int64_t m0, int mt) {                                 \
        const x86_weight *w = c->w;                                                                             \
        int64_t kb = w->kb;                                                                                     \
        __m256 acc[MAX_MT][2];                                                                                  \
        for (int i = 0; i < MAX_MT; i++) acc[i][0] = acc[i][1] = _mm256_setzero_ps();                           \
        for (int64_t b = 0; b < kb; b++) {                                                                      \
            if (w->type == OR_Q8_0) {                                                                           \
                const x86_act_q8_0 *acts[MAX_MT];                                                               \
                for (int i = 0; i < mt; i++) acts[i] = (const x86_act_q8_0 *)c->lhs_q + (m0 + i) * kb + b;      \
                const x86_tile_q8_0 *t = (const x86_tile_q8_0 *)w->tiles + nt * kb * 8 + b * 8;                 \
                for (int s = 0; s < 8; s += 2) Q80(t + s, t + s + 1, acts, mt, s, acc);                         \
            } else {                                                                                            \
                const or_block_q8k *acts[MAX_MT];                                                               \
                for (int i = 0; i < mt; i++) acts[i] = (const or_block_q8k *)c->lhs_q + (m0 + i) * kb + b;      \
                if (w->type == OR_Q4K) Q4K((const x86_tile_q4k *)w->tiles + nt * kb + b, acts, mt, acc);        \
                else Q6K((const x86_tile_q6k *)w->tiles + nt * kb + b, acts, mt, acc);                          \
            }                                                                                                   \
        }                                                                                                       \
        for (int i = 0; i < mt; i++) {                                                                          \
            _mm256_storeu_ps(c->dst + (m0 + i) * w->n + nt * TILE_N, acc[i][0]);                                \
            _mm256_storeu_ps(c->dst + (m0 + i) * w->n + nt * TILE_N + 8, acc[i][1]);                            \
        }                                                                                                       \
    }
UNIT_256(unit_avx2, T256, q4k_tile_avx2, q6k_tile_avx2, q8_0_tile2_avx2)
UNIT_256(unit_avxvnni, T256V, q4k_tile_avxvnni, q6k_tile_avxvnni, q8_0_tile2_avxvnni)

/* matmul_tiles: units are (16-column tile, MAX_MT activation rows), the row blocks fastest */
static void tiles_range(void *vctx, int64_t begin, int64_t end) {
    const tiles_ctx *c = vctx;
    int64_t m_units = (c->m + MAX_MT - 1) / MAX_MT;
    for (int64_t u = begin; u < end; u++) {
        int64_t nt = u / m_units, m0 = (u % m_units) * MAX_MT;
        int mt = (int)(c->m - m0 < MAX_MT ? c->m - m0 : MAX_MT);
        if (c->level == X86_AVX512VNNI) unit_512(c, nt, m0, mt);
        else if (c->level == X86_AVXVNNI) unit_avxvnni(c, nt, m0, mt);
        else unit_avx2(c, nt, m0, mt);
    }
}

/* ------------------------------------------------------------------ AMX, Q4_K at m >= 32 (repack_x86.rs:1068-1303) */

#define TAMX __attribute__((target("avx512f,avx512bw,amx-tile,amx-int8,fma")))

typedef struct {
    uint8_t palette, start_row, rsvd[14];
    uint16_t colsb[16];
    uint8_t rows[16];
} __attribute__((aligned(64))) amx_cfg;

/* tmm0-3: C (16x16 i32); tmm4-5: A (16 rows x 32 i8); tmm6-7: B (8 rows x 64 i8), loaded once per thread */
static _Thread_local int amx_ready;

TAMX static void amx_configure(void) {
    if (amx_ready) return;
    amx_cfg cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.palette = 1;
    for (int t = 0; t < 4; t++) { cfg.colsb[t] = 64; cfg.rows[t] = 16; }
    for (int t = 4; t < 6; t++) { cfg.colsb[t] = 32; cfg.rows[t] = 16; }
    for (int t = 6; t < 8; t++) { cfg.colsb[t] = 64; cfg.rows[t] = 8; }
    _tile_loadconfig(&cfg);
    amx_ready = 1;
}

typedef struct { const x86_weight *w; const or_block_q8k *lhs_q; int64_t m; float *dst; } amx_ctx;

/* q4k_m32: 32 activation rows x 32 weight columns per step, 4 C tiles from 2 A and 2 B loads per sub-block;
 * each sub-block's 16x16 integer tiles are scaled into an f32 accumulator at once */
TAMX static void amx_q4k_m32(const amx_ctx *c, const int8_t *a_pack, int64_t m0, int mt, int64_t nt0) {
    const x86_weight *w = c->w;
    int64_t kb = w->kb, n_tiles = w->n / TILE_N, a_half = kb * 8 * 16 * 32;
    int two_n = nt0 + 1 < n_tiles;
    const x86_tile_q4k_amx *tiles = w->amx_tiles;
    int32_t cs[4 * 16 * 16] __attribute__((aligned(64)));
    float facc[32 * 32] __attribute__((aligned(64)));
    memset(facc, 0, sizeof facc);
    for (int64_t b = 0; b < kb; b++) {
        const x86_tile_q4k_amx *t0 = &tiles[nt0 * kb + b], *t1 = &tiles[(nt0 + two_n) * kb + b];
        for (int sub = 0; sub < 8; sub++) {
            const int8_t *a0 = a_pack + (b * 8 + sub) * 16 * 32, *a1 = a_pack + a_half + (b * 8 + sub) * 16 * 32;
            _tile_zero(0);
            _tile_zero(1);
            _tile_zero(2);
            _tile_zero(3);
            _tile_loadd(4, a0, 32);
            _tile_loadd(6, t0->qs + sub * 8 * TILE_N * 4, 64);
            _tile_dpbssd(0, 4, 6);
            _tile_loadd(7, t1->qs + sub * 8 * TILE_N * 4, 64);
            _tile_dpbssd(1, 4, 7);
            _tile_loadd(5, a1, 32);
            _tile_dpbssd(2, 5, 6);
            _tile_dpbssd(3, 5, 7);
            _tile_stored(0, cs, 64);
            _tile_stored(1, cs + 256, 64);
            _tile_stored(2, cs + 512, 64);
            _tile_stored(3, cs + 768, 64);
            for (int half = 0; half < 2; half++) {
                int rows = half == 0 ? (mt < 16 ? mt : 16) : (mt > 16 ? mt - 16 : 0);
                for (int ntl = 0; ntl < 1 + two_n; ntl++) {
                    const x86_tile_q4k_amx *tile = ntl ? t1 : t0;
                    __m512 scale = _mm512_loadu_ps(tile->scales[sub]), min = _mm512_loadu_ps(tile->mins[sub]);
                    int cbase = (half * 2 + ntl) * 256;
                    for (int mi = 0; mi < rows; mi++) {
                        const or_block_q8k *act = &c->lhs_q[(m0 + half * 16 + mi) * kb + b];
                        float dall = act->d;
                        __m512 cf = _mm512_cvtepi32_ps(_mm512_loadu_si512(cs + cbase + mi * 16));
                        float *fp = facc + (half * 16 + mi) * 32 + ntl * 16;
                        float bsum = (float)((int32_t)act->bsums[sub * 2] + (int32_t)act->bsums[sub * 2 + 1]);
                        __m512 f = _mm512_fmadd_ps(cf, _mm512_mul_ps(scale, _mm512_set1_ps(dall)), _mm512_loadu_ps(fp));
                        f = _mm512_fnmadd_ps(min, _mm512_set1_ps(dall * bsum), f);
                        _mm512_storeu_ps(fp, f);
                    }
                }
            }
        }
    }
    int n_cols = 16 * (1 + two_n);
    for (int mi = 0; mi < mt; mi++)
        memcpy(c->dst + (m0 + mi) * w->n + nt0 * TILE_N, facc + mi * 32, (size_t)n_cols * sizeof(float));
}

/* matmul_amx_q4k: ranges of 32-row activation blocks; each thread repacks its block's activations as
 * [half][superblock][sub-block][16 rows][32 bytes] and walks every pair of weight tiles */
TAMX static void amx_range(void *vctx, int64_t begin, int64_t end) {
    const amx_ctx *c = vctx;
    amx_configure();
    int64_t kb = c->w->kb, a_half = kb * 8 * 16 * 32, n_tiles = c->w->n / TILE_N;
    int8_t *a_pack = aligned_alloc(64, (size_t)(2 * a_half));
    for (int64_t mb = begin; mb < end; mb++) {
        int64_t m0 = mb * 32;
        int mt = (int)(c->m - m0 < 32 ? c->m - m0 : 32);
        memset(a_pack, 0, (size_t)(2 * a_half));
        for (int i = 0; i < mt; i++) {
            int8_t *base = a_pack + (i / 16) * a_half;
            int r = i % 16;
            for (int64_t b = 0; b < kb; b++) {
                const int8_t *qs = c->lhs_q[(m0 + i) * kb + b].qs;
                for (int sub = 0; sub < 8; sub++) memcpy(base + ((b * 8 + sub) * 16 + r) * 32, qs + sub * 32, 32);
            }
        }
        for (int64_t nt = 0; nt < n_tiles; nt += 2) amx_q4k_m32(c, a_pack, m0, mt, nt);
    }
    free(a_pack);
}

/* ------------------------------------------------------------------ compact AVX2 path (k_quants.rs:2776-2894, avx.rs) */

/* vec_dot_q6k_q8k (avx.rs:212-303): per 128 values, the 6-bit values rebuilt from ql/qh, maddubs against the
 * activations minus 32x their maddubs against 32, scaled per 16 values by the signed scales, summed in i32 */
T256 static float vec_dot_q6k_avx2(int64_t nb, const or_block_q6k *x, const or_block_q8k *y) {
    const __m256i m4 = _mm256_set1_epi8(0xF), m2 = _mm256_set1_epi8(3), m32s = _mm256_set1_epi8(32);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < nb; i++) {
        float d = y[i].d * oracle_f16_to_f32(x[i].d);
        const uint8_t *q4 = x[i].ql, *qh = x[i].qh;
        const int8_t *q8 = y[i].qs;
        __m128i scales = _mm_loadu_si128((const __m128i *)x[i].scales);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 2; j++) {
            __m256i sc[4];
            for (int s = 0; s < 4; s++) {
                /* bytes 2(4j+s) and 2(4j+s)+1 of the scales, each repeated eight times (scale of 16 values) */
                int lo = 2 * (4 * j + s);
                __m128i shuf = _mm_setr_epi8(lo, lo, lo, lo, lo, lo, lo, lo, lo + 1, lo + 1, lo + 1, lo + 1, lo + 1,
                                             lo + 1, lo + 1, lo + 1);
                sc[s] = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, shuf));
            }
            __m256i b1 = _mm256_loadu_si256((const __m256i *)q4), b2 = _mm256_loadu_si256((const __m256i *)(q4 + 32));
            __m256i bh = _mm256_loadu_si256((const __m256i *)qh);
            q4 += 64;
            qh += 32;
            __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(bh, m2), 4);
            __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 2), m2), 4);
            __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 4), m2), 4);
            __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 6), m2), 4);
            __m256i v[4] = {_mm256_or_si256(_mm256_and_si256(b1, m4), h0), _mm256_or_si256(_mm256_and_si256(b2, m4), h1),
                            _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b1, 4), m4), h2),
                            _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b2, 4), m4), h3)};
            for (int s = 0; s < 4; s++) {
                __m256i a = _mm256_loadu_si256((const __m256i *)(q8 + 32 * s));
                __m256i p = _mm256_sub_epi16(_mm256_maddubs_epi16(v[s], a), _mm256_maddubs_epi16(m32s, a));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(sc[s], p));
            }
            q8 += 128;
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    __m128 r = _mm_add_ps(_mm256_extractf128_ps(acc, 1), _mm256_castps256_ps128(acc));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}

/* vec_dot_q8_0_q8_0 (avx.rs:110-127): per block f32(dx)*f32(dy) times the i8 x i8 dot as floats (the sign of x
 * moved onto y for maddubs) */
T256 static float vec_dot_q8_0_avx2(int64_t nb, const or_block_q8_0 *x, const or_block_q8_0 *y) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int64_t i = 0; i < nb; i++) {
        __m256 d = _mm256_set1_ps(oracle_f16_to_f32(x[i].d) * oracle_f16_to_f32(y[i].d));
        __m256i bx = _mm256_loadu_si256((const __m256i *)x[i].qs), by = _mm256_loadu_si256((const __m256i *)y[i].qs);
        __m256i ax = _mm256_sign_epi8(bx, bx), sy = _mm256_sign_epi8(by, bx);
        __m256 q = _mm256_cvtepi32_ps(_mm256_madd_epi16(ones, _mm256_maddubs_epi16(ax, sy)));
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    __m128 r = _mm_add_ps(_mm256_extractf128_ps(acc, 1), _mm256_castps256_ps128(acc));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}

typedef struct { const x86_weight *w; const void *lhs_row; float *dst_row; } compact_ctx;

static void compact_range(void *vctx, int64_t begin, int64_t end) {
    const compact_ctx *c = vctx;
    const x86_weight *w = c->w;
    for (int64_t col = begin; col < end; col++) {
        if (w->type == OR_Q6K)
            c->dst_row[col] = vec_dot_q6k_avx2(w->kb, (const or_block_q6k *)w->blocks + col * w->kb, c->lhs_row);
        else
            c->dst_row[col] = vec_dot_q8_0_avx2(w->k / OR_QK8_0, (const or_block_q8_0 *)w->blocks + col * (w->k / OR_QK8_0),
                                                c->lhs_row);
    }
}

/* ------------------------------------------------------------------ QMatMul forward on x86 */

/* The reference's CPU QMatMul on this host: repack::try_matmul_f32 (repack.rs:232-262) when select() takes the
 * shape (AMX for Q4_K at m >= 32 where available, else the tiles at the detected level), otherwise
 * k_quants::matmul with the AVX2 vec_dot (Q6_K and Q8_0 at m = 1), otherwise the scalar oracle.
 * dst is [m][n] f32.  threads <= 0 uses the physical cores.  Returns the path taken (1 AMX, 2 tiles, 3 compact
 * AVX2, 4 scalar) or -1 on an error. */
int oracle_x86_matmul(const void *handle, int64_t m, const float *lhs, float *dst, int threads) {
    const x86_weight *w = handle;
    if (!w || m <= 0) return -1;
    int T = threads > 0 ? threads : oracle_x86_physical_cores();
    int64_t kb = w->kb, n = w->n, k = w->k;
    int lv = oracle_x86_level();
    if (w->tiles && oracle_x86_select(w->type, m, n, k)) {
        int q8_0 = w->type == OR_Q8_0;
        size_t act = q8_0 ? sizeof(x86_act_q8_0) : sizeof(or_block_q8k);
        void *lhs_q = aligned_alloc(64, (size_t)(m * kb) * act);
        if (!lhs_q) return -1;
        quant_ctx qc = {lhs, k, kb, lhs_q, q8_0};
        if (m == 1) quant_rows(&qc, 0, 1);
        else run_ranges(T, m, 0, quant_rows, &qc);
        int path;
        if (!q8_0 && m >= 32 && w->type == OR_Q4K && w->amx_tiles && oracle_x86_amx()) {
            amx_ctx ac = {w, lhs_q, m, dst};
            run_ranges(T, (m + 31) / 32, 0, amx_range, &ac);
            path = 1;
        } else {
            tiles_ctx tc = {w, lhs_q, m, dst, lv};
            run_ranges(T, (n / TILE_N) * ((m + MAX_MT - 1) / MAX_MT), 0, tiles_range, &tc);
            path = 2;
        }
        free(lhs_q);
        return path;
    }
    if ((w->type == OR_Q6K || w->type == OR_Q8_0) && lv != X86_NONE) {
        int q8_0 = w->type == OR_Q8_0;
        int64_t blocks = q8_0 ? k / OR_QK8_0 : kb;
        size_t act = q8_0 ? sizeof(or_block_q8_0) : sizeof(or_block_q8k);
        void *row_q = aligned_alloc(64, (size_t)blocks * act + 64);
        if (!row_q) return -1;
        for (int64_t r = 0; r < m; r++) {
            if (q8_0) oracle_quantize_q8_0(lhs + r * k, k, row_q);
            else oracle_quantize_q8k(lhs + r * k, k, row_q);
            compact_ctx cc = {w, row_q, dst + r * n};
            /* Q6_K at m = 1 splits its equal dot products statically (k_quants.rs:2865-2871) */
            run_ranges(T, n, w->type == OR_Q6K && m == 1, compact_range, &cc);
        }
        free(row_q);
        return 3;
    }
    return oracle_matmul(w->type, m, k, n, lhs, w->blocks, dst, T) == 0 ? 4 : -1;
}

/* "<model name> (<level>[, AMX])" for reports */
int oracle_x86_describe(char *buf, int len) {
    char model[256] = "unknown CPU";
    FILE *f = fopen("/proc/cpuinfo", "r");
    if (f) {
        char line[512];
        while (fgets(line, sizeof line, f)) {
            if (strncmp(line, "model name", 10) == 0) {
                char *p = strchr(line, ':');
                if (p) {
                    p++;
                    while (*p == ' ' || *p == '\t') p++;
                    snprintf(model, sizeof model, "%s", p);
                    model[strcspn(model, "\n")] = 0;
                }
                break;
            }
        }
        fclose(f);
    }
    static const char *names[] = {"no AVX2", "AVX2", "AVX-VNNI", "AVX-512 VNNI"};
    return snprintf(buf, (size_t)len, "%s (%s%s)", model, names[oracle_x86_level()], oracle_x86_amx() ? ", AMX" : "");
}
