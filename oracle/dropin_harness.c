/* SPDX-License-Identifier: Apache-2.0 */
/*
 * dropin_harness.c - a C caller of the drop-in k3_kda_layer, built against the REFERENCE's
 * own header (include/k3/k3.h, for K3Cfg, K3KdaW and the prototypes) and linked to
 * libk3kda_hip.so instead of the reference's k3_ops.c: the link-time substitution an engine
 * makes to run its KDA layers on the GPU. TEST INFRASTRUCTURE ONLY (tests/test_gpu_dropin.py
 * runs it); it mirrors the reference's t_kda_layer (tests/unit/test_ops.c:576-634): zeroed
 * structs, a state array of H*D*D + 3*P*(conv_k-1) floats, scratch sized by k3_kda_scratch,
 * then k3_kda_layer.
 *
 * Usage: dropin_harness DIR
 *   DIR/case.txt   "hidden H D conv_k wdt gate_lb rms_eps ncalls T_1 .. T_ncalls state0"
 *                  (state0 = 1: DIR/state_in.bin holds the initial state, else zeros)
 *   DIR/<name>.bin the weights of K3KdaW as raw bytes (q k v q_conv k_conv v_conv f_a f_b
 *                  A_log dt_bias b g o_norm o), in the storage their wdt tag names
 *   DIR/x<i>.bin   call i's input [T_i][hidden] fp32
 * Writes DIR/out<i>.bin ([T_i][hidden] fp32) and DIR/state<i>.bin (the whole state after
 * call i). Exit status 0 on success.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "k3.h"

static void *slurp(const char *dir, const char *name, size_t *n)
{
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", dir, name);
    FILE *f = fopen(p, "rb");
    if (!f) {
        fprintf(stderr, "dropin_harness: cannot open %s\n", p);
        exit(2);
    }
    fseek(f, 0, SEEK_END);
    const long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *buf = malloc(len > 0 ? (size_t)len : 1);
    if (!buf || (len > 0 && fread(buf, 1, (size_t)len, f) != (size_t)len)) {
        fprintf(stderr, "dropin_harness: cannot read %s\n", p);
        exit(2);
    }
    fclose(f);
    if (n) *n = (size_t)len;
    return buf;
}

static void spill(const char *dir, const char *name, const void *p, size_t bytes)
{
    char path[1024];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "dropin_harness: cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

int main(int argc, char **argv)
{
    if (argc != 2) {
        fprintf(stderr, "usage: %s DIR\n", argv[0]);
        return 2;
    }
    const char *dir = argv[1];
    char *txt = (char *)slurp(dir, "case.txt", NULL);
    int hidden, H, D, K, wdt, ncalls, state0 = 0, Ts[64];
    float lb, eps;
    int used = 0;
    if (sscanf(txt, "%d %d %d %d %d %f %f %d%n", &hidden, &H, &D, &K, &wdt, &lb, &eps, &ncalls, &used) != 8 ||
        ncalls < 1 || ncalls > 64) {
        fprintf(stderr, "dropin_harness: bad case.txt\n");
        return 2;
    }
    char *at = txt + used;
    for (int i = 0; i < ncalls; i++) {
        int u = 0;
        if (sscanf(at, "%d%n", &Ts[i], &u) != 1 || Ts[i] < 1) {
            fprintf(stderr, "dropin_harness: bad T list\n");
            return 2;
        }
        at += u;
    }
    if (sscanf(at, "%d", &state0) != 1) state0 = 0;

    K3Cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = hidden;
    c.kda_heads = H;
    c.kda_head_dim = D;
    c.conv_k = K;
    c.gate_lb = lb;
    c.rms_eps = eps;

    K3KdaW w;
    memset(&w, 0, sizeof w);
    w.q = slurp(dir, "q.bin", NULL);
    w.k = slurp(dir, "k.bin", NULL);
    w.v = slurp(dir, "v.bin", NULL);
    w.q_conv = (const float *)slurp(dir, "q_conv.bin", NULL);
    w.k_conv = (const float *)slurp(dir, "k_conv.bin", NULL);
    w.v_conv = (const float *)slurp(dir, "v_conv.bin", NULL);
    w.f_a = slurp(dir, "f_a.bin", NULL);
    w.f_b = slurp(dir, "f_b.bin", NULL);
    w.A_log = (const float *)slurp(dir, "A_log.bin", NULL);
    w.dt_bias = (const float *)slurp(dir, "dt_bias.bin", NULL);
    w.b = slurp(dir, "b.bin", NULL);
    w.g = slurp(dir, "g.bin", NULL);
    w.o_norm = (const float *)slurp(dir, "o_norm.bin", NULL);
    w.o = slurp(dir, "o.bin", NULL);
    w.wdt = wdt;

    const size_t P = (size_t)H * D;
    const size_t nst = P * D + 3 * P * (size_t)(K - 1);
    float *st = (float *)calloc(nst, sizeof(float));
    if (!st) return 2;
    if (state0) {
        size_t n = 0;
        float *s0 = (float *)slurp(dir, "state_in.bin", &n);
        if (n != nst * sizeof(float)) {
            fprintf(stderr, "dropin_harness: state_in.bin has %zu bytes, want %zu\n", n, nst * sizeof(float));
            return 2;
        }
        memcpy(st, s0, n);
        free(s0);
    }
    for (int i = 0; i < ncalls; i++) {
        const int T = Ts[i];
        char nm[64];
        size_t n = 0;
        snprintf(nm, sizeof nm, "x%d.bin", i);
        float *x = (float *)slurp(dir, nm, &n);
        if (n != (size_t)T * hidden * sizeof(float)) {
            fprintf(stderr, "dropin_harness: %s has %zu bytes\n", nm, n);
            return 2;
        }
        float *sc = (float *)malloc(k3_kda_scratch(&c, T) * sizeof(float));
        float *y = (float *)malloc((size_t)T * hidden * sizeof(float));
        if (!sc || !y) return 2;
        k3_kda_layer(y, x, &w, &c, T, st, sc);
        snprintf(nm, sizeof nm, "out%d.bin", i);
        spill(dir, nm, y, (size_t)T * hidden * sizeof(float));
        snprintf(nm, sizeof nm, "state%d.bin", i);
        spill(dir, nm, st, nst * sizeof(float));
        free(x);
        free(sc);
        free(y);
        printf("call %d: T=%d done\n", i, T);
    }
    return 0;
}
