/* abi_host.c -- a plain C host of libhymt_hip.so: the calls a non-Python
 * binding (the C# HipBackend's P/Invoke layer, IComputeBackend.cs:14-88)
 * makes for one layer's attention, through include/hymt_hip.h only.
 *
 *   abi_host IN OUT
 *
 * IN holds int32 heads, kv_heads, head_dim, pos, seq, kv_dtype, then fp32
 * gamma_q[D], gamma_k[D], bf16 cache rows k[pos][kv_heads*D], v[...] (the
 * model's flat caches, UploadKv's layout), fp32 prefill rows q[seq][heads*D],
 * k[seq][kv_heads*D], v[...], and fp32 decode rows q[heads*D], k[kv_heads*D],
 * v[...].  The program uploads the cache, runs a prefill of `seq` tokens at
 * `pos` and a decode at pos + seq (host pointers), and writes the prefill
 * output [seq][heads*D] then the decode output [heads*D] (fp32) to OUT.
 *
 * Exit status: 0 done; 3 no HIP device (the library loaded and the device
 * probe answered); 4 the error path misbehaved (a NULL context must return
 * an error code with a message); 1 any other failure, with the library's
 * message on stderr.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "hymt_hip.h"

static int fail(const char *what, int code) {
    fprintf(stderr, "abi_host: %s failed (%d): %s\n", what, code, hymt_last_error());
    return 1;
}

#define CALL(expr)                          \
    do {                                    \
        int rc_ = (expr);                   \
        if (rc_ != HYMT_OK) return fail(#expr, rc_); \
    } while (0)

static void *read_n(FILE *f, size_t bytes) {
    void *p = malloc(bytes ? bytes : 1);
    if (p && bytes && fread(p, 1, bytes, f) != bytes) {
        free(p);
        return NULL;
    }
    return p;
}

static int run(FILE *in, FILE *out) {
    int32_t hdr[6];
    if (fread(hdr, sizeof hdr, 1, in) != 1) return fail("reading the header", -1);
    const int heads = hdr[0], kv_heads = hdr[1], D = hdr[2], pos = hdr[3], seq = hdr[4], kv_dtype = hdr[5];
    const size_t qd = (size_t)heads * D, kd = (size_t)kv_heads * D;
    float *qnw = read_n(in, D * sizeof(float)), *knw = read_n(in, D * sizeof(float));
    uint16_t *kc = read_n(in, (size_t)pos * kd * 2), *vc = read_n(in, (size_t)pos * kd * 2);
    float *pq = read_n(in, seq * qd * 4), *pk = read_n(in, seq * kd * 4), *pv = read_n(in, seq * kd * 4);
    float *dq = read_n(in, qd * 4), *dk = read_n(in, kd * 4), *dv = read_n(in, kd * 4);
    float *pout = malloc(seq * qd * 4 + 4), *dout = malloc(qd * 4);
    if (!qnw || !knw || !kc || !vc || !pq || !pk || !pv || !dq || !dk || !dv || !pout || !dout)
        return fail("reading the inputs", -1);

    /* the error path: a NULL context is refused with a message */
    if (hymt_attn_decode(NULL, 0, 0, dq, dk, dv, NULL, NULL, dout, 0) == HYMT_OK || !hymt_last_error()[0]) {
        fprintf(stderr, "abi_host: a NULL context was not refused\n");
        return 4;
    }
    int count = 0;
    CALL(hymt_device_count(&count));
    if (count < 1) {
        printf("no HIP device\n");
        return 3;
    }
    hymt_ctx *ctx = NULL;
    CALL(hymt_create(0, &ctx));
    CALL(hymt_set_attn_config(ctx, heads, kv_heads, D, D, 10000.0f, 1e-6f));
    CALL(hymt_kv_create(ctx, 1, pos + seq + 1, kv_dtype));
    if (pos > 0) CALL(hymt_kv_upload(ctx, 0, 0, pos, kc, vc));
    CALL(hymt_attn_prefill(ctx, 0, pos, seq, pq, pk, pv, HYMT_F32, qnw, knw, pout, 0));
    CALL(hymt_attn_decode(ctx, 0, pos + seq, dq, dk, dv, qnw, knw, dout, 0));
    CALL(hymt_sync(ctx));
    CALL(hymt_destroy(ctx));
    if (fwrite(pout, 4, seq * qd, out) != seq * qd || fwrite(dout, 4, qd, out) != qd)
        return fail("writing the outputs", -1);
    free(qnw); free(knw); free(kc); free(vc); free(pq); free(pk); free(pv);
    free(dq); free(dk); free(dv); free(pout); free(dout);
    return 0;
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: abi_host IN OUT\n");
        return 1;
    }
    FILE *in = fopen(argv[1], "rb");
    if (!in) return fail("opening IN", -1);
    FILE *out = fopen(argv[2], "wb");
    if (!out) return fail("opening OUT", -1);
    const int rc = run(in, out);
    fclose(in);
    if (fclose(out) != 0 && rc == 0) return fail("closing OUT", -1);
    return rc;
}
