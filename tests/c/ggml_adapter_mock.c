/* Compiles include/mxfa_ggml.h against a mock struct ggml_tensor (the
 * fields the adapter reads, in ggml's order) and prints the descriptors it
 * derives from a flash-attention node, plus mxfa_supports()'s verdict, and
 * the set_rows adapter's verdicts on a KV-cache write node.
 * Built and run by tests/test_ggml_adapter.py. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#define MOCK_MAX_SRC 10
struct ggml_tensor {
    int type;                                  /* enum ggml_type */
    void *buffer;
    int64_t ne[4];
    size_t nb[4];
    int op;                                    /* never read by the adapter */
    int32_t op_params[64 / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor *src[MOCK_MAX_SRC];
    struct ggml_tensor *view_src;
    size_t view_offs;
    void *data;
    char name[64];
    void *extra;
};

#include "mxfa_ggml.h"

static void set4(int64_t *ne, int64_t a, int64_t b, int64_t c, int64_t d) { ne[0] = a; ne[1] = b; ne[2] = c; ne[3] = d; }

static void contig(struct ggml_tensor *t, size_t esz) {
    t->nb[0] = esz;
    for (int i = 1; i < 4; i++) t->nb[i] = t->nb[i - 1] * (size_t)t->ne[i - 1];
}

static void show(const char *name, const mxfa_tensor *d) {
    if (!d) { printf("%s NULL\n", name); return; }
    printf("%s type=%d ne=%lld,%lld,%lld,%lld nb=%zu,%zu,%zu,%zu data=%p\n", name, d->type,
           (long long)d->ne[0], (long long)d->ne[1], (long long)d->ne[2], (long long)d->ne[3],
           d->nb[0], d->nb[1], d->nb[2], d->nb[3], d->data);
}

int main(int argc, char **argv) {
    const int with_mask = argc > 1 && strcmp(argv[1], "mask") == 0;
    const int with_sinks = argc > 1 && strcmp(argv[1], "sinks") == 0;
    struct ggml_tensor q, k, v, m, node, sinks;
    memset(&q, 0, sizeof q); memset(&k, 0, sizeof k); memset(&v, 0, sizeof v);
    memset(&m, 0, sizeof m); memset(&node, 0, sizeof node); memset(&sinks, 0, sizeof sinks);
    /* batched CFG decode view (src/qwen3-lm.h:780-794): q [128,1,32,8] permuted,
     * k/v [128, 8192, 8, 8] F16 cache views, mask [8192, 1, 1, 8] F16 */
    q.type = 0; set4(q.ne, 128, 1, 32, 8); q.nb[0] = 4; q.nb[1] = 4 * 128 * 32; q.nb[2] = 4 * 128; q.nb[3] = 4 * 128 * 32;
    q.data = (void *)(uintptr_t)0x100000;
    k.type = 1; set4(k.ne, 128, 8192, 8, 8); k.nb[0] = 2; k.nb[1] = 256; k.nb[2] = 256 * 8192; k.nb[3] = 256 * 8192 * 8;
    k.data = (void *)(uintptr_t)0x200000;
    v = k; v.data = (void *)(uintptr_t)0x300000;
    m.type = 1; set4(m.ne, 8192, 1, 1, 8); contig(&m, 2); m.data = (void *)(uintptr_t)0x400000;
    node.type = 0; set4(node.ne, 128, 32, 1, 8); contig(&node, 4); node.data = (void *)(uintptr_t)0x500000;
    node.op = 12345;   /* arbitrary: the adapter does not look at it */
    node.src[0] = &q; node.src[1] = &k; node.src[2] = &v; node.src[3] = with_mask ? &m : NULL;
    if (with_sinks) node.src[4] = &sinks;
    const float params[3] = {0.08838834764831845f, 0.0f, 0.0f};
    const int32_t prec = 10;   /* GGML_PREC_F32 */
    memcpy(node.op_params, params, sizeof params);
    memcpy((char *)node.op_params + 3 * sizeof(float), &prec, sizeof prec);

    mxfa_tensor dq, dk, dv, dm, dd;
    const mxfa_tensor *mp = NULL;
    mxfa_params p;
    const int rc = mxfa_ggml_unpack(&node, &dq, &dk, &dv, &dm, &mp, &dd, &p);
    printf("unpack %d\n", rc);
    if (rc == 0) {
        show("q", &dq); show("k", &dk); show("v", &dv); show("mask", mp); show("dst", &dd);
        printf("params scale=%.9g max_bias=%g softcap=%g prec=%d\n", p.scale, p.max_bias, p.logit_softcap, p.prec);
    }
    printf("supports %d\n", mxfa_ggml_supports(&node));

    /* the KV-cache write before it (src/qwen3-lm.h:760-777): node = view of
     * the [128, 8192, 8, 8] F16 cache sets, src[0] = F32 [128, 1, 8, 8] rows,
     * src[1] = I64 [1, 1, 8] positions */
    struct ggml_tensor sr, kn, ids;
    memset(&sr, 0, sizeof sr); memset(&kn, 0, sizeof kn); memset(&ids, 0, sizeof ids);
    sr = k; sr.src[0] = &kn; sr.src[1] = &ids;
    kn.type = 0; set4(kn.ne, 128, 1, 8, 8); contig(&kn, 4); kn.data = (void *)(uintptr_t)0x600000;
    ids.type = 27; set4(ids.ne, 1, 1, 8, 1); contig(&ids, 8); ids.data = (void *)(uintptr_t)0x700000;
    printf("set_rows_supports %d\n", mxfa_ggml_set_rows_supports(&sr));
    ids.type = 28;   /* F64: not a row-id type */
    printf("set_rows_bad_ids %d\n", mxfa_ggml_set_rows_supports(&sr));
    sr.src[1] = NULL;
    printf("set_rows_no_ids %d %d\n", mxfa_ggml_set_rows_supports(&sr), mxfa_ggml_set_rows(&sr, NULL));

    /* the pre-attention step of a 4B-LM layer as one custom node
     * (src/qwen3-lm.h:418-454): 7 tokens, 32 / 8 heads, 2048-slot caches */
    struct ggml_tensor nq, nk, nv, qw, kw, pos, ck, cv, rid, qo;
    struct ggml_tensor *all[] = {&nq, &nk, &nv, &qw, &kw, &pos, &ck, &cv, &rid, &qo};
    for (int i = 0; i < 10; i++) memset(all[i], 0, sizeof *all[i]);
    nq.type = 0; set4(nq.ne, 128, 32, 7, 1); contig(&nq, 4); nq.data = (void *)(uintptr_t)0x800000;
    nk.type = 0; set4(nk.ne, 128, 8, 7, 1); contig(&nk, 4); nk.data = (void *)(uintptr_t)0x900000;
    nv = nk; nv.data = (void *)(uintptr_t)0xA00000;
    qw.type = 0; set4(qw.ne, 128, 1, 1, 1); contig(&qw, 4); qw.data = (void *)(uintptr_t)0xB00000;
    kw = qw; kw.data = (void *)(uintptr_t)0xB10000;
    pos.type = 26; set4(pos.ne, 7, 1, 1, 1); contig(&pos, 4); pos.data = (void *)(uintptr_t)0xC00000;
    ck.type = 1; set4(ck.ne, 128, 2048, 8, 1); contig(&ck, 2); ck.data = (void *)(uintptr_t)0xD00000;
    cv = ck; cv.data = (void *)(uintptr_t)0xE00000;
    rid.type = 27; set4(rid.ne, 7, 1, 1, 1); contig(&rid, 8); rid.data = (void *)(uintptr_t)0xF00000;
    qo.type = 1; set4(qo.ne, 128, 32, 7, 1); contig(&qo, 2); qo.data = (void *)(uintptr_t)0x1000000;
    qo.src[0] = &nq; qo.src[1] = &nk; qo.src[2] = &nv; qo.src[3] = &qw; qo.src[4] = &kw;
    qo.src[5] = &pos; qo.src[6] = &ck; qo.src[7] = &cv; qo.src[8] = &rid;
    const mxfa_norm_rope_params np = {1e-6f, 1000000.0f, 0};
    mxfa_tensor nt[10];
    const mxfa_tensor *nrows = NULL;
    printf("nr_unpack %d\n", mxfa_ggml_unpack_norm_rope(&qo, nt, &nrows));
    show("nr_q", &nt[0]); show("nr_kcache", &nt[6]); show("nr_qout", &nt[8]); show("nr_rows", nrows);
    printf("nr_supports %d\n", mxfa_ggml_qk_norm_rope_supports(&qo, &np));
    pos.type = 27;   /* I64 positions: the rope positions are I32 */
    printf("nr_bad_pos %d\n", mxfa_ggml_qk_norm_rope_supports(&qo, &np));
    pos.type = 26;
    qo.src[8] = NULL;   /* no row ids: row s of the caches */
    printf("nr_no_rows %d\n", mxfa_ggml_qk_norm_rope_supports(&qo, &np));
    qo.src[6] = NULL;
    printf("nr_no_cache %d %d\n", mxfa_ggml_qk_norm_rope_supports(&qo, &np), mxfa_ggml_qk_norm_rope(&qo, &np, NULL));
    return 0;
}
