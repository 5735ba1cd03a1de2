/* layout_probe.c - prints sizeof/offsetof of K3Cfg, K3KdaW and K3MlaW. TEST INFRASTRUCTURE.
 * Built twice by oracle/Makefile: once against the reference include/k3/k3.h and once
 * (-DMIRROR) against include/k3kda.h; the two outputs must be identical. */
#include <stddef.h>
#include <stdio.h>
#ifdef MIRROR
#include "k3kda.h"
#else
#include "k3.h"
#endif

#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m))

int main(void)
{
    printf("K3Cfg %zu\n", sizeof(K3Cfg));
    F(K3Cfg, hidden); F(K3Cfg, rms_eps); F(K3Cfg, kda_heads); F(K3Cfg, kda_head_dim);
    F(K3Cfg, conv_k); F(K3Cfg, gate_lb); F(K3Cfg, mla_out_gate); F(K3Cfg, routed_scale);
    F(K3Cfg, attn_res_block); F(K3Cfg, situ_b2); F(K3Cfg, n_full_attn); F(K3Cfg, full_attn);
    printf("K3KdaW %zu\n", sizeof(K3KdaW));
    F(K3KdaW, q); F(K3KdaW, k); F(K3KdaW, v); F(K3KdaW, q_conv); F(K3KdaW, k_conv);
    F(K3KdaW, v_conv); F(K3KdaW, f_a); F(K3KdaW, f_b); F(K3KdaW, A_log);
    F(K3KdaW, dt_bias); F(K3KdaW, b); F(K3KdaW, g); F(K3KdaW, o_norm); F(K3KdaW, o);
    F(K3KdaW, wdt);
    printf("K3MlaW %zu\n", sizeof(K3MlaW));
    F(K3MlaW, q_a); F(K3MlaW, q_b); F(K3MlaW, kv_a); F(K3MlaW, kv_b); F(K3MlaW, o);
    F(K3MlaW, g); F(K3MlaW, q_a_norm); F(K3MlaW, kv_a_norm); F(K3MlaW, wdt);
    return 0;
}
