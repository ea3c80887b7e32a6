/* sc_oracle.c - CPU restatement of the reference's prefill->decode cache handoff.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this
 * library, and only as the checker or the timed CPU baseline.  The product (libsc_handoff.so) never links,
 * loads or calls it, and has no CPU fallback.
 *
 * Every function names the reference code it restates.  Pinning (what each one is checked against, so that a
 * dropped term, a wrong index or a transposed operand fails a test):
 *   sco_f16_bits            the reference's numpy-generated f32->f16 vectors (src/kernels/qsa_oracle_vectors.inc,
 *                           committed as tests/golden/f16_oracle_vectors.json) and numpy astype(float16)
 *   sco_kv_append           numpy reshape/transpose of [T][H][D] into [page][H][ps][D] and the two rival layouts of
 *                           src/kernels/qsa_parity.cpp:489-497, which must differ
 *   sco_rec_carve           numpy transpose(1, 0, 2) and the fused_gdn.cu:31-33 index form
 *   sco_conv_hist           numpy qkv[T-3:T].T, and the T < 3 cases against an explicit history shift
 *   sco_image_layout        the published payload totals (59 899 904 / 884 342 784 / 3 300 261 888 bytes)
 *                           and the closed forms cells = ceil(T/4)*4, data = cells*H*D*2
 *   sco_park / sco_resume   A/B/A round trips and byte accounting
 *   sco_fnv1a64             textbook FNV-1a 64 vectors with the standard basis; the reference's seed on empty input
 *   sco_fill_*              the device generators of libsc_handoff.so, bit for bit (GPU tests), and moments
 *   sco_synth_*_hash        sco_fnv1a64 over the outputs of sco_fill_* -> sco_kv_append / sco_rec_carve /
 *                           sco_conv_hist -> sco_park on small sequences (one and two sources per blob)
 *   sco_f32_of_f16          numpy float16 -> float32 on all 65536 bit patterns
 *   sco_q8_row / sco_q4_row numpy vectorised restatements of the same rules (independent of these loops) on random and
 *                           edge groups (zero, tied magnitudes, exact .5 quotients, clamping, tiny and huge scales),
 *                           plus hand-computed blocks
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Same field order as sc_geometry (include/sc_handoff.h) and strata::core::ModelGeometry's subset. */
typedef struct sco_geometry {
    int64_t n_layers, qsa_interval, n_head_kv, head_dim, page_size;
    int64_t ssm_state_size, ssm_k_heads, ssm_v_heads, ssm_d_conv, ssm_conv_channels, idx_key_dim;
} sco_geometry;

/* ---- synthetic inputs ----------------------------------------------------------------------------------------- */

uint64_t sco_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t sco_synth_key(uint64_t seed, uint64_t sid) { return sco_mix64(seed ^ sco_mix64(sid + 0x9E3779B97F4A7C15ull)); }

static uint64_t draw(uint64_t key, uint64_t i) { return sco_mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

/* ---- f32 -> f16 ------------------------------------------------------------------------------------------------ */

/* Round to nearest even, from the IEEE-754 binary16 definition.  NaN -> sign|0x7C00|0x200 and finite overflow ->
 * infinity, the conventions of include/strata/kernels/f16_bits.hpp:37-70 (the reference's decode-side
 * converter).  Written as exact rational rounding on the mantissa as an integer: the value is m * 2^(e-23);
 * the f16 result keeps floor(m / 2^k) with k = 13 for normals and k = 14 - e16 in the subnormal range. */
uint16_t sco_f16_bits(uint32_t x) {
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e8 = (int) ((x >> 23) & 0xFFu);
    uint32_t m = x & 0x7FFFFFu;
    if (e8 == 0xFF) return (uint16_t) (sign | 0x7C00u | (m ? 0x200u : 0u));
    if (e8 == 0) return (uint16_t) sign;             /* f32 subnormals are far below the f16 range: +-0 */
    m |= 0x800000u;                                   /* value = m * 2^(e8 - 150) */
    const int e16 = e8 - 127 + 15;                    /* biased f16 exponent if normal */
    int k = e16 >= 1 ? 13 : 14 - e16;                 /* mantissa bits dropped */
    if (k > 24) return (uint16_t) sign;               /* below half the smallest subnormal */
    uint32_t q = m >> k;
    const uint32_t rem = m - (q << k), half = 1u << (k - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    /* q counts units of the last place: 2^(e16-25) for normals (with the implicit bit at 2^10), 2^-24 below */
    uint32_t bits;
    if (e16 >= 1) {
        uint32_t e = (uint32_t) e16;
        if (q == 0x800u) { q = 0x400u; ++e; }        /* rounding carried into the next binade */
        if (e >= 31) return (uint16_t) (sign | 0x7C00u);
        bits = (e << 10) | (q & 0x3FFu);
    } else {
        bits = q;                                     /* q == 0x400 is the smallest normal, encoded the same way */
    }
    return (uint16_t) (sign | bits);
}

void sco_f16_from_f32(const float* src, uint16_t* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t x;
        memcpy(&x, &src[i], 4);
        dst[i] = sco_f16_bits(x);
    }
}

void sco_fill_uniform_f32(float* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t sid) {
    const uint64_t key = sco_synth_key(seed, sid);
    const float span = hi - lo;
    for (uint64_t i = 0; i < n; ++i) {
        const float u = (float) (uint32_t) (draw(key, i) >> 40) * 0x1p-24f;
        dst[i] = fmaf(span, u, lo);
    }
}

void sco_fill_uniform_f16(uint16_t* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t sid) {
    const uint64_t key = sco_synth_key(seed, sid);
    const float span = hi - lo;
    for (uint64_t i = 0; i < n; ++i) {
        const float u = (float) (uint32_t) (draw(key, i) >> 40) * 0x1p-24f;
        const float x = fmaf(span, u, lo);
        uint32_t b;
        memcpy(&b, &x, 4);
        dst[i] = sco_f16_bits(b);
    }
}

/* Irwin-Hall(12) - 6: mean 0, variance 1, formed in integers so every platform gets the same bits. */
void sco_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t sid) {
    const uint64_t key = sco_synth_key(seed, sid);
    for (uint64_t i = 0; i < n; ++i) {
        int64_t sum = 0;
        for (int k = 0; k < 6; ++k) {
            const uint64_t x = draw(key, i * 6 + (uint64_t) k);
            sum += (int64_t) (x >> 40) + (int64_t) ((x >> 16) & 0xFFFFFFull);
        }
        dst[i] = (float) (int32_t) (sum - ((int64_t) 6 << 24)) * 0x1p-24f;
    }
}

/* ---- the carve -------------------------------------------------------------------------------------------------- */

/* kv_append (src/prefill/kernels.cu:560-601, launched at :618-625): token t of kv head h, element d, goes to cell
 * pos = pos0 + t at pool[((table[pos/ps] * H + h) * ps + pos % ps) * D + d]; a page that is not resident
 * (negative entry) is skipped, as kernels.cu:577 skips it.  `src` is f16 bits (dtype 0) or f32 (dtype 1, rounded
 * to f16 as kernels.cu:575 rounds it).  Entries at or past n_pages are skipped too (the device never writes past
 * its pool). */
void sco_kv_append(const void* src, int dtype, int64_t T, int64_t pos0, const int32_t* table, int64_t n_pages,
                   int64_t H, int64_t D, int64_t ps, uint16_t* pool) {
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < H; ++h) {
            const int64_t pos = pos0 + t;
            const int64_t page = table ? (int64_t) table[pos / ps] : pos / ps;
            if (page < 0 || page >= n_pages) continue;
            const int64_t row = (page * H + h) * ps + pos % ps;
            for (int64_t d = 0; d < D; ++d) {
                const int64_t i = (t * H + h) * D + d;
                uint16_t v;
                if (dtype == 0) {
                    v = ((const uint16_t*) src)[i];
                } else {
                    uint32_t b;
                    memcpy(&b, (const float*) src + i, 4);
                    v = sco_f16_bits(b);
                }
                pool[row * D + d] = v;
            }
        }
}

/* ---- quantized K/V formats ------------------------------------------------------------------------------------- */

/* binary16 bits -> binary32, exactly (every f16 value is an f32 value). */
float sco_f32_of_f16(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) bits = sign | 0x7F800000u | (m << 13);
    else if (e) bits = sign | ((e + 112u) << 23) | (m << 13);
    else if (!m) bits = sign;
    else {   /* subnormal: normalise */
        int shift = 0;
        uint32_t mm = m;
        while (!(mm & 0x400u)) { mm <<= 1; ++shift; }
        bits = sign | ((uint32_t) (113 - shift) << 23) | ((mm & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* int8 K/V: the reference's int8 kv_append (src/prefill/kernels.cu:578-600) and kv_append_q8
 * (src/kernels/cuda/kv_q8.cu:29-64), whose host restatement is src/kernels/kv_q8_parity.cpp:78-92.  Per group of 64
 * values: amax = max |x| over the values that are not NaN (the device writers' fmaxf reduction passes a NaN over);
 * the stored scale is f16(amax / 127) rounded to nearest even; each code is rint(x / f32(scale)) (ties to even)
 * clamped to [-127, 127], or 0 when the scale is 0.  A NaN value gets code 0 (the reference leaves NaN undefined).  A
 * group of NaNs only reduces to NaN there, so its scale is f16 NaN, 0x7E00 under the reference's converter
 * (f16_bits.hpp:37-70, |NaN| being positive), and every code 0.  `codes` gets D bytes, `scales` D/64 f16 words. */
void sco_q8_row(const float* x, int64_t D, int8_t* codes, uint16_t* scales) {
    for (int64_t g = 0; g < D / 64; ++g) {
        const float* v = x + g * 64;
        float amax = 0.0f;                              /* NaNs never count toward the maximum */
        int real = 0;
        for (int t = 0; t < 64; ++t) {   /* any NaN, quiet or signalling, is passed over (CUDA's fmaxf rule) */
            const int is_real = v[t] == v[t];
            if (is_real && fabsf(v[t]) > amax) amax = fabsf(v[t]);
            real |= is_real;
        }
        const float ratio = amax / 127.0f;
        uint32_t rb;
        memcpy(&rb, &ratio, 4);
        const uint16_t sb = real ? sco_f16_bits(rb) : (uint16_t) 0x7E00u;
        const float sf = sco_f32_of_f16(sb);
        scales[g] = sb;
        for (int t = 0; t < 64; ++t) {
            int q = 0;                                  /* a NaN quotient converts to 0 (CUDA's float->int rule) */
            if (sf > 0.0f && v[t] == v[t]) {
                const float r = rintf(v[t] / sf);
                q = r != r ? 0 : (r < -127.0f ? -127 : (r > 127.0f ? 127 : (int) r));
            }
            codes[g * 64 + t] = (int8_t) q;
        }
    }
}

/* q4_0 K/V: kv_append_q4 (src/kernels/cuda/kv_q4.cu:72-89 q4_group, :111-129), host restatement
 * src/kernels/kv_q4_parity.cpp:64-87.  Per block of 32 values: the value of largest |x| (ties go to the larger value,
 * the device kernel's rule); d = that value / -8; id = 1/d (0 when d is 0); each code is trunc(x*id + 8.5) with one
 * rounding, a fused multiply-add (the device writer's form: kv_q4.cu:84 is contracted to an FMA by nvcc's default
 * --fmad=true and by clang's HIP default; the host checker rounds the product first), clamped to [0, 15]; byte j is
 * code j | code j+16 << 4; the block is {f16(d) RNE, 16 bytes} = 18 bytes.  Among values equal in magnitude and in
 * value (only +0 and -0 can be), the first in index order is the maximum, so the sign of a zero d is defined.
 * `blocks` gets D/32 * 18 bytes. */
void sco_q4_row(const float* x, int64_t D, uint8_t* blocks) {
    for (int64_t b = 0; b < D / 32; ++b) {
        const float* v = x + b * 32;
        /* NaN never compares larger, so it is never picked (the host form's rule, kv_q4_parity.cpp:68-73); a block
         * of NaNs keeps the start value +0.  Among equals the first index stays. */
        float amax = -1.0f, mval = 0.0f;
        for (int t = 0; t < 32; ++t) {
            const float a = fabsf(v[t]);
            if (a > amax || (a == amax && v[t] > mval)) { amax = a; mval = v[t]; }
        }
        const float d = mval / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t q[32];
        for (int t = 0; t < 32; ++t) {
            const float sum = fmaf(v[t], id, 8.5f);      /* one rounding, as the device writer's FMA */
            /* truncation toward zero saturating, as __float2int_rz does: an infinite sum (id overflows for a block
             * whose d is subnormal) clamps to 0 or 15, a NaN one (inf * 0) codes 0 */
            const float c = sum != sum ? 0.0f : (sum < 0.0f ? 0.0f : (sum > 15.0f ? 15.0f : sum));
            q[t] = (uint8_t) (int) c;
        }
        uint32_t db;
        memcpy(&db, &d, 4);
        const uint16_t dh = sco_f16_bits(db);
        uint8_t* blk = blocks + b * 18;
        blk[0] = (uint8_t) dh;
        blk[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < 16; ++j) blk[2 + j] = (uint8_t) (q[j] | (q[j + 16] << 4));
    }
}

/* The quantizing kv_append: f32 rows [T][H][D] (for q4_0 already rotated, as the reference rotates before
 * kv_append_q4) into a codes pool [page][H][ps][row_bytes] (row_bytes = D for int8, D/32*18 for q4_0) and, for int8,
 * a scale pool [page][H][ps][D/64] f16, through the page table like sco_kv_append. fmt: 1 int8, 2 q4_0. */
void sco_kv_append_quant(const float* src, int fmt, int64_t T, int64_t pos0, const int32_t* table, int64_t n_pages,
                         int64_t H, int64_t D, int64_t ps, uint8_t* codes, uint16_t* scales) {
    const int64_t row_bytes = fmt == 1 ? D : D / 32 * 18;
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < H; ++h) {
            const int64_t pos = pos0 + t;
            const int64_t page = table ? (int64_t) table[pos / ps] : pos / ps;
            if (page < 0 || page >= n_pages) continue;
            const int64_t row = (page * H + h) * ps + pos % ps;
            const float* x = src + (t * H + h) * D;
            if (fmt == 1) sco_q8_row(x, D, (int8_t*) codes + row * row_bytes, scales + row * (D / 64));
            else sco_q4_row(x, D, codes + row * row_bytes);
        }
}

/* The recurrence: element (i, h, j) of a head-major [HV][S][S] prefill image goes to i*HV*S + h*S + j, the
 * (S, HV, S) layout with j fastest that src/kernels/cuda/gdn.cu:75 and fused_gdn.cu:31-33 read and write. */
void sco_rec_carve(const float* src, int64_t S, int64_t HV, float* dst) {
    for (int64_t h = 0; h < HV; ++h)
        for (int64_t i = 0; i < S; ++i)
            for (int64_t j = 0; j < S; ++j) dst[(i * HV + h) * S + j] = src[(h * S + i) * S + j];
}

/* gdn_conv_hist_kernel (src/prefill/kernels.cu:219-228): after a chunk of `rows` input rows [rows][C] (row stride
 * ld), history slot k (of nhist) is input row rows - nhist + k, or - for a chunk shorter than the history - the
 * previous history's slot k + rows, read before any slot is overwritten.  A fresh sequence's previous history is
 * zero (session_zero / qsa_state_zero, include/strata/core/session.hpp:104, layer.hpp:306). */
void sco_conv_hist(float* hist, const float* qkv, int64_t rows, int64_t ld, int64_t C, int64_t nhist, int fresh) {
    float v[8];
    for (int64_t c = 0; c < C; ++c) {
        for (int64_t k = 0; k < nhist; ++k) {
            const int64_t t = rows - nhist + k;
            v[k] = t >= 0 ? qkv[t * ld + c] : fresh ? 0.0f : hist[c * nhist + (t + nhist)];
        }
        for (int64_t k = 0; k < nhist; ++k) hist[c * nhist + k] = v[k];
    }
}

/* ---- the image: a SavedConversation's K/V + GDN payload in blob-pool order ------------------------------------ */

typedef struct sco_blob {
    int32_t kind, layer;   /* 1 K, 2 V, 3 GDN */
    uint64_t offset, bytes;
} sco_blob;

static int64_t n_qsa(const sco_geometry* g) { return g->n_layers / g->qsa_interval; }
static int64_t n_gdn(const sco_geometry* g) { return g->n_layers - n_qsa(g); }
int64_t sco_gdn_row_floats(const sco_geometry* g) {
    return g->ssm_state_size * g->ssm_v_heads * g->ssm_state_size + g->ssm_conv_channels * (g->ssm_d_conv - 1);
}
/* conversation_snapshot.cpp:40: the page-granular extent a park copies. */
int64_t sco_cells(const sco_geometry* g, int64_t tokens) {
    return (tokens + g->page_size - 1) / g->page_size * g->page_size;
}

static uint64_t align64(uint64_t x) { return (x + 63) / 64 * 64; }

/* Blob order of the wire codec's pool (src/core/conversation_wire.cpp:400-437): every KV record's buffers in
 * kv order (k then v; f16 has no scale buffers), then the live checkpoint's gdn buffer; 64-byte aligned.
 * Sizes: data = cells * n_head_kv * head_dim * 2 (conversation_snapshot.cpp:40-49); gdn = n_gdn rows of
 * (S*HV*S + C*(d_conv-1)) floats (conversation_state.cpp:186-189). Returns the blob count. */
int64_t sco_image_layout(const sco_geometry* g, int64_t tokens, sco_blob* out, uint64_t* total) {
    const uint64_t kv = (uint64_t) sco_cells(g, tokens) * (uint64_t) g->n_head_kv * (uint64_t) g->head_dim * 2;
    uint64_t at = 0;
    int64_t n = 0;
    for (int64_t j = 0; j < n_qsa(g); ++j)
        for (int kind = 1; kind <= 2; ++kind) {
            at = align64(at);
            if (out) { out[n].kind = kind; out[n].layer = (int32_t) j; out[n].offset = at; out[n].bytes = kv; }
            ++n;
            at += kv;
        }
    if (n_gdn(g) > 0) {
        const uint64_t bytes = (uint64_t) n_gdn(g) * (uint64_t) sco_gdn_row_floats(g) * 4;
        at = align64(at);
        if (out) { out[n].kind = 3; out[n].layer = -1; out[n].offset = at; out[n].bytes = bytes; }
        ++n;
        at += bytes;
    }
    if (total) *total = align64(at);
    return n;
}

/* conversation_kv_save (src/core/conversation_snapshot.cpp:139-173) for identity-layout f16 pools: each buffer's
 * first `data` bytes, which are the first cells/ps pages; plus conversation_checkpoint_save's gdn copy
 * (conversation_state.cpp:233-235).  Host pointers; gaps in the image are zeroed. */
void sco_park(const sco_geometry* g, int64_t tokens, const uint16_t* const* k_pool, const uint16_t* const* v_pool,
              const float* gdn_state, uint8_t* image) {
    sco_blob blobs[4096];
    uint64_t total = 0;
    const int64_t n = sco_image_layout(g, tokens, blobs, &total);
    memset(image, 0, total);
    for (int64_t b = 0; b < n; ++b) {
        const void* from = blobs[b].kind == 3 ? (const void*) gdn_state
                         : blobs[b].kind == 1 ? (const void*) k_pool[blobs[b].layer] : (const void*) v_pool[blobs[b].layer];
        memcpy(image + blobs[b].offset, from, blobs[b].bytes);
    }
}

/* conversation_kv_restore (conversation_snapshot.cpp:196-204) + conversation_checkpoint_restore's gdn copy
 * (conversation_state.cpp:251): the inverse of sco_park. */
void sco_resume(const sco_geometry* g, int64_t tokens, const uint8_t* image, uint16_t* const* k_pool,
                uint16_t* const* v_pool, float* gdn_state) {
    sco_blob blobs[4096];
    uint64_t total = 0;
    const int64_t n = sco_image_layout(g, tokens, blobs, &total);
    for (int64_t b = 0; b < n; ++b) {
        void* to = blobs[b].kind == 3 ? (void*) gdn_state
                 : blobs[b].kind == 1 ? (void*) k_pool[blobs[b].layer] : (void*) v_pool[blobs[b].layer];
        memcpy(to, image + blobs[b].offset, blobs[b].bytes);
    }
}

/* ---- FNV-1a 64 ----------------------------------------------------------------------------------------------- */

/* src/core/pinned.cu:594-601: xor the byte, then multiply by the 64-bit FNV prime.  The reference seeds every call
 * with 1469598103934665603 = 0x14650fb0739d0383 (conversation_snapshot.cpp:225, conversation_wire.hpp:196), not
 * the textbook basis 0xcbf29ce484222325; callers pass the seed. */
uint64_t sco_fnv1a64(const uint8_t* p, uint64_t n, uint64_t seed) {
    uint64_t h = seed;
    for (uint64_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

/* ---- whole-blob hashes of synthetic sequences -------------------------------------------------------------------
 * The FNV-1a of one blob of the image a synthetic sequence carves to, generated value by value from the counter-based
 * generators (sco_fill_*) and folded into the hash as it goes, so the full-size configs (up to 3.3 GB of payload) are
 * compared with the device byte for byte without materialising the expected bytes.  The layouts are the ones
 * sco_kv_append, sco_rec_carve, sco_conv_hist and sco_image_layout restate: a K/V blob is the identity pool's first
 * `cells` cells ([page][H][ps][D] f16, conversation_snapshot.cpp:40-49), the GDN blob is every GDN row
 * ((S, HV, S) recurrence then the [C][d_conv-1] history, conversation_state.cpp:186-189).  Pinned by the tests against
 * sco_fnv1a64 over those functions' outputs (fill -> carve -> park) on small sequences, single and two-source. */

/* One source of a K/V blob: cells [t0, t0 + n) hold tokens 0 .. n-1 of a synthetic sequence whose K (or V) rows are
 * element (t * H + h) * D + d of stream `sid` under `seed`, U[lo, hi] rounded to f16 (sco_fill_uniform_f16; an f32
 * source rounded by the carve gives the same bits, sco_fill_uniform_f32 then sco_f16_bits). */
typedef struct sco_kv_source {
    uint64_t seed, sid;
    int64_t t0, n;
    float lo, hi;
} sco_kv_source;

static uint64_t fnv_byte(uint64_t h, uint8_t b) { return (h ^ b) * 1099511628211ull; }

uint64_t sco_synth_kv_blob_hash(int64_t H, int64_t D, int64_t ps, int64_t cells, const sco_kv_source* src,
                                int32_t n_src, uint8_t tail, uint64_t fnv_seed) {
    uint64_t h = fnv_seed;
    uint64_t keys[8];
    for (int32_t s = 0; s < n_src && s < 8; ++s) keys[s] = sco_synth_key(src[s].seed, src[s].sid);
    for (int64_t page = 0; page * ps < cells; ++page)
        for (int64_t kh = 0; kh < H; ++kh)
            for (int64_t c = 0; c < ps; ++c) {
                const int64_t cell = page * ps + c;
                int32_t s = 0;
                while (s < n_src && !(cell >= src[s].t0 && cell < src[s].t0 + src[s].n)) ++s;
                if (s == n_src || s >= 8) {
                    for (int64_t d = 0; d < D; ++d) h = fnv_byte(fnv_byte(h, tail), tail);
                    continue;
                }
                const uint64_t base = (uint64_t) (((cell - src[s].t0) * H + kh) * D);
                const float span = src[s].hi - src[s].lo;
                for (int64_t d = 0; d < D; ++d) {
                    const float u = (float) (uint32_t) (draw(keys[s], base + (uint64_t) d) >> 40) * 0x1p-24f;
                    const float x = fmaf(span, u, src[s].lo);
                    uint32_t b;
                    memcpy(&b, &x, 4);
                    const uint16_t v = sco_f16_bits(b);
                    h = fnv_byte(fnv_byte(h, (uint8_t) v), (uint8_t) (v >> 8));
                }
            }
    return h;
}

/* One blob of a quantized slot a synthetic f32 sequence carves to (the quantizing kv_append of every token, identity
 * pool): `fmt` 1 int8 or 2 q4_0, `part` 0 the codes pool ([page][H][ps][row] bytes: D int8 codes or D/32 q4_0 blocks of
 * 18 bytes) or 1 the int8 scales ([page][H][ps][D/64] f16), over the first `cells` cells; row (t, h) quantizes element
 * (t * H + h) * D + d of stream `sid` under `seed`, U[lo, hi] in f32 (sco_fill_uniform_f32) with sco_q8_row or
 * sco_q4_row, and the rows of cells at or past `tokens` hold `tail` bytes. */
uint64_t sco_synth_quant_blob_hash(int64_t H, int64_t D, int64_t ps, int64_t cells, uint64_t seed, uint64_t sid,
                                   int64_t tokens, float lo, float hi, int32_t fmt, int32_t part, uint8_t tail,
                                   uint64_t fnv_seed) {
    if (D > 1024 || D % 64) return 0;
    const uint64_t key = sco_synth_key(seed, sid);
    const float span = hi - lo;
    const int64_t row_bytes = part == 1 ? D / 64 * 2 : fmt == 1 ? D : D / 32 * 18;
    float x[1024];
    uint8_t out[1024];
    uint16_t scales[16];
    uint64_t h = fnv_seed;
    for (int64_t page = 0; page * ps < cells; ++page)
        for (int64_t kh = 0; kh < H; ++kh)
            for (int64_t c = 0; c < ps; ++c) {
                const int64_t t = page * ps + c;
                if (t >= tokens) {
                    for (int64_t b = 0; b < row_bytes; ++b) h = fnv_byte(h, tail);
                    continue;
                }
                const uint64_t base = (uint64_t) ((t * H + kh) * D);
                for (int64_t d = 0; d < D; ++d) {
                    const float u = (float) (uint32_t) (draw(key, base + (uint64_t) d) >> 40) * 0x1p-24f;
                    x[d] = fmaf(span, u, lo);
                }
                const uint8_t* bytes = out;
                if (fmt == 1) {
                    sco_q8_row(x, D, (int8_t*) out, scales);
                    if (part == 1) bytes = (const uint8_t*) scales;
                } else {
                    sco_q4_row(x, D, out);
                }
                for (int64_t b = 0; b < row_bytes; ++b) h = fnv_byte(h, bytes[b]);
            }
    return h;
}

static float normal_at(uint64_t key, uint64_t i) {
    int64_t sum = 0;
    for (int k = 0; k < 6; ++k) {
        const uint64_t x = draw(key, i * 6 + (uint64_t) k);
        sum += (int64_t) (x >> 40) + (int64_t) ((x >> 16) & 0xFFFFFFull);
    }
    return (float) (int32_t) (sum - ((int64_t) 6 << 24)) * 0x1p-24f;
}

static uint64_t fnv_f32(uint64_t h, float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    for (int k = 0; k < 4; ++k) h = fnv_byte(h, (uint8_t) (b >> (8 * k)));
    return h;
}

/* The GDN blob of a sequence carved fresh (pos0 = 0): GDN layer i's recurrence is stream sid_rec0 + i, head-major
 * [HV][S][S] N(0,1) (sco_fill_normal_f32), carved to (S, HV, S); its history is the last d_conv-1 of `conv_rows`
 * rows of stream sid_conv0 + i ([rows][C], row stride C), rows before the first reading as zero. */
uint64_t sco_synth_gdn_hash(const sco_geometry* g, uint64_t seed, uint64_t sid_rec0, uint64_t sid_conv0,
                            int64_t conv_rows, uint64_t fnv_seed) {
    const int64_t S = g->ssm_state_size, HV = g->ssm_v_heads, Cc = g->ssm_conv_channels, nh = g->ssm_d_conv - 1;
    uint64_t h = fnv_seed;
    for (int64_t i = 0; i < n_gdn(g); ++i) {
        const uint64_t kr = sco_synth_key(seed, sid_rec0 + (uint64_t) i);
        const uint64_t kc = sco_synth_key(seed, sid_conv0 + (uint64_t) i);
        for (int64_t a = 0; a < S; ++a)
            for (int64_t hv = 0; hv < HV; ++hv)
                for (int64_t b = 0; b < S; ++b) h = fnv_f32(h, normal_at(kr, (uint64_t) ((hv * S + a) * S + b)));
        for (int64_t c = 0; c < Cc; ++c)
            for (int64_t k = 0; k < nh; ++k) {
                const int64_t t = conv_rows - nh + k;
                h = fnv_f32(h, t >= 0 ? normal_at(kc, (uint64_t) (t * Cc + c)) : 0.0f);
            }
    }
    return h;
}

/* ---- the whole handoff, as the CPU would do it --------------------------------------------------------------- */

/* The fused carve of one sequence into a decode slot (identity or paged pools), host pointers: what
 * sc_plan_carve computes.  Layer arrays are in QSA / GDN order. */
void sco_handoff_carve(const sco_geometry* g, int64_t T, int64_t pos0, int dtype, const void* const* k_src,
                       const void* const* v_src, int with_gdn, const float* const* rec_src,
                       const float* const* conv_src, int64_t conv_rows, int64_t conv_ld,
                       uint16_t* const* k_pool, uint16_t* const* v_pool, const int32_t* const* tables,
                       int64_t n_pages, float* gdn_state) {
    for (int64_t j = 0; j < n_qsa(g); ++j) {
        const int32_t* table = tables ? tables[j] : NULL;
        sco_kv_append(k_src[j], dtype, T, pos0, table, n_pages, g->n_head_kv, g->head_dim, g->page_size, k_pool[j]);
        sco_kv_append(v_src[j], dtype, T, pos0, table, n_pages, g->n_head_kv, g->head_dim, g->page_size, v_pool[j]);
    }
    if (!with_gdn) return;
    const int64_t row = sco_gdn_row_floats(g), S = g->ssm_state_size, HV = g->ssm_v_heads;
    for (int64_t i = 0; i < n_gdn(g); ++i) {
        float* base = gdn_state + i * row;
        sco_rec_carve(rec_src[i], S, HV, base);
        sco_conv_hist(base + S * HV * S, conv_src[i], conv_rows, conv_ld, g->ssm_conv_channels, g->ssm_d_conv - 1,
                      pos0 == 0);
    }
}

/* The reference's host-side handoff of an already-parked image, restated as the CPU baseline:
 *   save    - conversation_kv_save's copy into 16 MiB segments (include/strata/core/conversation_buffer.hpp:18,
 *             conversation_snapshot.cpp:160-171): one segment buffer per <=16 MiB piece of each blob;
 *   encode  - the wire codec's blob pool with FNV-1a over every written byte (conversation_wire.cpp:400-480);
 *   decode  - copy out of the payload into fresh segments and re-check the hash (conversation_wire.cpp:694-754,
 *             handoff.cpp:1133-1136);
 *   restore - conversation_kv_restore's copy back into the slot (conversation_snapshot.cpp:196-204).
 * `slot_src` and `slot_dst` are contiguous images of the slot's payload (as sco_park lays it out); `scratch`
 * must hold 3 * image bytes.  Returns the payload hash (the caller compares encode and decode hashes through
 * the return values of two calls, or trusts the internal check: a mismatch returns 0). */
uint64_t sco_cpu_handoff(const uint8_t* slot_src, uint8_t* slot_dst, uint64_t bytes, uint8_t* scratch) {
    const uint64_t seg = 16ull << 20;
    const uint64_t seed = 1469598103934665603ull;
    uint8_t* saved = scratch;
    uint8_t* wire = scratch + bytes;
    uint8_t* decoded = scratch + 2 * bytes;
    for (uint64_t at = 0; at < bytes; at += seg) memcpy(saved + at, slot_src + at, bytes - at < seg ? bytes - at : seg);
    uint64_t h_enc = seed;
    for (uint64_t at = 0; at < bytes; at += seg) {
        const uint64_t n = bytes - at < seg ? bytes - at : seg;
        memcpy(wire + at, saved + at, n);
        h_enc = sco_fnv1a64(wire + at, n, h_enc);
    }
    const uint64_t h_dec = sco_fnv1a64(wire, bytes, seed);
    if (h_dec != h_enc) return 0;
    for (uint64_t at = 0; at < bytes; at += seg) memcpy(decoded + at, wire + at, bytes - at < seg ? bytes - at : seg);
    for (uint64_t at = 0; at < bytes; at += seg) memcpy(slot_dst + at, decoded + at, bytes - at < seg ? bytes - at : seg);
    return h_enc;
}

/* Not the reference's path: the host's plain copy ceiling for the CPU baseline's labelled N-core variant.  `threads`
 * threads each memcpy one contiguous 1/threads share of `bytes` (at 4 KiB granules) from src to dst. */
typedef struct {
    uint8_t* dst;
    const uint8_t* src;
    uint64_t n;
} sco_copy_share;

static void* sco_copy_worker(void* arg) {
    const sco_copy_share* s = (const sco_copy_share*) arg;
    memcpy(s->dst, s->src, s->n);
    return NULL;
}

int sco_memcpy_threads(uint8_t* dst, const uint8_t* src, uint64_t bytes, int threads) {
    enum { kMaxThreads = 64 };
    if (threads < 1 || threads > kMaxThreads) return -1;
    pthread_t tid[kMaxThreads];
    sco_copy_share share[kMaxThreads];
    const uint64_t per = ((bytes / (uint64_t) threads) + 4095) & ~4095ull;
    int started = 0;
    for (int i = 0; i < threads; ++i) {
        const uint64_t at = per * (uint64_t) i;
        share[i].dst = dst + at;
        share[i].src = src + at;
        share[i].n = at >= bytes ? 0 : (bytes - at < per ? bytes - at : per);
        if (i == 0) continue;   /* the calling thread takes share 0 */
        if (pthread_create(&tid[i], NULL, sco_copy_worker, &share[i]) != 0) break;
        started = i;
    }
    sco_copy_worker(&share[0]);
    for (int i = 1; i <= started; ++i) pthread_join(tid[i], NULL);
    if (started != threads - 1) {   /* a thread could not start: copy its shares here */
        for (int i = started + 1; i < threads; ++i) sco_copy_worker(&share[i]);
    }
    return 0;
}
