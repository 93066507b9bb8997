/*
 * CPU restatement of the reference's adaptive (de Casteljau) flattening and
 * its CSR gradient accumulation.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (repo_amd/, manbo/) may
 * link, load or call this file; only tests/ use it, always as the checker.
 *
 * Arithmetic spec: fp32, IEEE + - * / sqrt in the reference's expression
 * order, no implicit contraction (-ffp-contract=off).  The subdivision is
 * restated the way the reference runs it -- level by level over arrays of
 * active cubics, leaves gathered per level, then one sort by (segment, t0)
 * -- so that it checks the GPU's left-to-right walk independently.
 *
 * Reference files followed (under /root/reference/manbo/ops/):
 *   cubic_splatting.py:1729-1832 _flatten_cubics_to_edges (de Casteljau branch)
 *                                -> orc_flatten_decas
 *   cubic_splatting.py:1863-1965 cubic_adaptive_flatness_flags_kernel / _tilelang
 *                                -> orc_cubic_flat, orc_flatness_flags
 *   cubic_splatting.py:1968-2068 cubic_split_half_kernel / _tilelang -> orc_split_half
 *   cubic_splatting.py:2399-2487 _accumulate_edge_grads_to_cubics_csr_kernel
 *                                -> orc_accumulate_edge_grads_csr
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_EPS ((float)1e-6)

/* cubic_splatting.py:1886-1913: the larger distance of P1, P2 from the chord
 * line; for a chord shorter than sqrt(1e-6) the largest of |P1-P0|, |P2-P0|,
 * |P3-P0|.  Flat when that is at most tol. */
int orc_cubic_flat(const float *c, float tol)
{
    float x0 = c[0], y0 = c[1], x1 = c[2], y1 = c[3];
    float x2 = c[4], y2 = c[5], x3 = c[6], y3 = c[7];
    float lx = x3 - x0, ly = y3 - y0;
    float chord2 = lx * lx + ly * ly;
    float chord = sqrtf(fmaxf(chord2, ORC_EPS));
    float v1x = x1 - x0, v1y = y1 - y0, v2x = x2 - x0, v2y = y2 - y0;
    float cross1 = fabsf(lx * v1y - ly * v1x);
    float cross2 = fabsf(lx * v2y - ly * v2x);
    float d1 = cross1 / chord, d2 = cross2 / chord;
    float dmax_line = fmaxf(d1, d2);
    float n1 = sqrtf(fmaxf(v1x * v1x + v1y * v1y, 0.0f));
    float n2 = sqrtf(fmaxf(v2x * v2x + v2y * v2y, 0.0f));
    float n3 = sqrtf(fmaxf(chord2, 0.0f));
    float dmax_degen = fmaxf(n1, fmaxf(n2, n3));
    float dmax = chord2 <= ORC_EPS ? dmax_degen : dmax_line;
    return dmax <= tol;
}

/* cubic_adaptive_flatness_flags_tilelang: tol clamped at 1e-4 (:1961). */
void orc_flatness_flags(const float *cubics, int32_t n, float tol, int32_t force, uint8_t *out)
{
    float t = fmaxf(1e-4f, tol);
    for (int32_t i = 0; i < n; ++i)
        out[i] = force ? 1 : (uint8_t)orc_cubic_flat(cubics + (size_t)i * 8, t);
}

/* cubic_split_half_kernel (cubic_splatting.py:1998-2028). */
static void orc_split_one(const float *c, float *l, float *r)
{
    for (int a = 0; a < 2; ++a) {
        float p0 = c[a], p1 = c[2 + a], p2 = c[4 + a], p3 = c[6 + a];
        float p01 = 0.5f * (p0 + p1);
        float p12 = 0.5f * (p1 + p2);
        float p23 = 0.5f * (p2 + p3);
        float p012 = 0.5f * (p01 + p12);
        float p123 = 0.5f * (p12 + p23);
        float p0123 = 0.5f * (p012 + p123);
        l[a] = p0; l[2 + a] = p01; l[4 + a] = p012; l[6 + a] = p0123;
        r[a] = p0123; r[2 + a] = p123; r[4 + a] = p23; r[6 + a] = p3;
    }
}

void orc_split_half(const float *cubics, int32_t n, float *left, float *right)
{
    for (int32_t i = 0; i < n; ++i)
        orc_split_one(cubics + (size_t)i * 8, left + (size_t)i * 8, right + (size_t)i * 8);
}

/* max_depth = ceil(log2(max(1, S - 1))) (cubic_splatting.py:1733). */
int32_t orc_decas_max_depth(int32_t S)
{
    int32_t eps = S - 1 > 1 ? S - 1 : 1;
    return (int32_t)ceil(log2((double)eps));
}

typedef struct {
    int64_t key;
    float p0x, p0y, p3x, p3y, t0, t1;
    int32_t sid;
} orc_leaf_t;

static int orc_leaf_cmp(const void *a, const void *b)
{
    int64_t ka = ((const orc_leaf_t *)a)->key, kb = ((const orc_leaf_t *)b)->key;
    return ka < kb ? -1 : (ka > kb ? 1 : 0);
}

/* cubic_splatting.py:1729-1832.  Writes up to cap edges [cap,2,2], their
 * t_starts / t_ends and seg_edge_offsets [nseg+1]; returns the edge count
 * (-1 if cap is too small or memory runs out). */
int32_t orc_flatten_decas(const float *cubics_px, int32_t nseg, int32_t S, float *edges,
                          float *t_starts, float *t_ends, int32_t *seg_edge_offsets,
                          int32_t cap)
{
    const float tol = fmaxf(1e-4f, 0.5f);   /* DEFAULT_DE_CASTELJAU_FLATNESS_TOL_PX */
    const int32_t max_depth = orc_decas_max_depth(S);
    const size_t most = (size_t)nseg << max_depth;
    float *cp = malloc(sizeof(float) * 8 * (most ? most : 1));
    float *cp2 = malloc(sizeof(float) * 8 * (most ? most : 1));
    int32_t *sid = malloc(sizeof(int32_t) * (most ? most : 1));
    int32_t *sid2 = malloc(sizeof(int32_t) * (most ? most : 1));
    float *a0 = malloc(sizeof(float) * (most ? most : 1));
    float *a1 = malloc(sizeof(float) * (most ? most : 1));
    float *b0 = malloc(sizeof(float) * (most ? most : 1));
    float *b1 = malloc(sizeof(float) * (most ? most : 1));
    orc_leaf_t *leaves = malloc(sizeof(orc_leaf_t) * (most ? most : 1));
    int32_t result = -1;
    if (!cp || !cp2 || !sid || !sid2 || !a0 || !a1 || !b0 || !b1 || !leaves) goto out;

    size_t n = (size_t)nseg, nleaf = 0;
    memcpy(cp, cubics_px, sizeof(float) * 8 * n);
    for (size_t i = 0; i < n; ++i) { sid[i] = (int32_t)i; a0[i] = 0.0f; a1[i] = 1.0f; }
    for (int32_t depth = 0; depth <= max_depth && n > 0; ++depth) {
        const int force = depth >= max_depth;
        /* leaves of this level, in active order (:1756-1762) */
        size_t nsplit = 0;
        for (size_t i = 0; i < n; ++i) {
            const float *c = cp + i * 8;
            if (force || orc_cubic_flat(c, tol)) {
                orc_leaf_t *L = leaves + nleaf++;
                L->p0x = c[0]; L->p0y = c[1]; L->p3x = c[6]; L->p3y = c[7];
                L->sid = sid[i]; L->t0 = a0[i]; L->t1 = a1[i];
            } else {
                ++nsplit;
            }
        }
        if (nsplit == 0) break;
        /* next level: all left halves, then all right halves (:1767-1781) */
        size_t j = 0;
        for (size_t i = 0; i < n; ++i) {
            const float *c = cp + i * 8;
            if (force || orc_cubic_flat(c, tol)) continue;
            float tmid = 0.5f * (a0[i] + a1[i]);
            orc_split_one(c, cp2 + j * 8, cp2 + (j + nsplit) * 8);
            sid2[j] = sid[i]; sid2[j + nsplit] = sid[i];
            b0[j] = a0[i]; b1[j] = tmid;
            b0[j + nsplit] = tmid; b1[j + nsplit] = a1[i];
            ++j;
        }
        n = 2 * nsplit;
        float *tf; int32_t *ti;
        tf = cp; cp = cp2; cp2 = tf;
        ti = sid; sid = sid2; sid2 = ti;
        tf = a0; a0 = b0; b0 = tf;
        tf = a1; a1 = b1; b1 = tf;
    }
    /* sort by sid * (2^D + 1) + round(t0 * 2^D) (:1801-1809) */
    const int64_t base = ((int64_t)1 << max_depth) + 1;
    for (size_t i = 0; i < nleaf; ++i) {
        double tok = nearbyint((double)(leaves[i].t0 * (float)(base - 1)));
        if (tok < 0) tok = 0;
        if (tok > (double)(base - 1)) tok = (double)(base - 1);
        leaves[i].key = (int64_t)leaves[i].sid * base + (int64_t)tok;
    }
    qsort(leaves, nleaf, sizeof(orc_leaf_t), orc_leaf_cmp);
    if ((int64_t)nleaf > cap) goto out;
    for (int32_t s = 0; s <= nseg; ++s) seg_edge_offsets[s] = 0;
    for (size_t i = 0; i < nleaf; ++i) {
        float *e = edges + i * 4;
        e[0] = leaves[i].p0x; e[1] = leaves[i].p0y; e[2] = leaves[i].p3x; e[3] = leaves[i].p3y;
        t_starts[i] = leaves[i].t0;
        t_ends[i] = leaves[i].t1;
        seg_edge_offsets[leaves[i].sid + 1] += 1;
    }
    for (int32_t s = 0; s < nseg; ++s) seg_edge_offsets[s + 1] += seg_edge_offsets[s];
    result = (int32_t)nleaf;
out:
    free(cp); free(cp2); free(sid); free(sid2); free(a0); free(a1); free(b0); free(b1);
    free(leaves);
    return result;
}

/* cubic_splatting.py:2432-2485: v_P_k = sum_e gs_e b_k(t0_e) + ge_e b_k(t1_e)
 * over the segment's CSR edge range; weights in fp32, sums in double. */
void orc_accumulate_edge_grads_csr(const double *v_edges, const int32_t *seo, const float *t0s,
                                   const float *t1s, int32_t nseg, double *v_cubics)
{
    for (int32_t s = 0; s < nseg; ++s) {
        double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int32_t e = seo[s]; e < seo[s + 1]; ++e) {
            float t0 = t0s[e], t1 = t1s[e];
            float o0 = 1.0f - t0, o1 = 1.0f - t1;
            float o0s = o0 * o0, o1s = o1 * o1, t0s2 = t0 * t0, t1s2 = t1 * t1;
            float b0[4] = {o0s * o0, 3.0f * o0s * t0, 3.0f * o0 * t0s2, t0s2 * t0};
            float b1[4] = {o1s * o1, 3.0f * o1s * t1, 3.0f * o1 * t1s2, t1s2 * t1};
            const double *g = v_edges + (size_t)e * 4;
            for (int k = 0; k < 4; ++k) {
                acc[2 * k] += g[0] * (double)b0[k] + g[2] * (double)b1[k];
                acc[2 * k + 1] += g[1] * (double)b0[k] + g[3] * (double)b1[k];
            }
        }
        memcpy(v_cubics + (size_t)s * 8, acc, sizeof(acc));
    }
}
