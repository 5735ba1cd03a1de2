// SPDX-License-Identifier: Apache-2.0
// kda_step.hip - one decode token of a whole KDA layer between its projections, for gfx950:
// K1 (short conv + SiLU, L2 norm, decay gate, beta), K3 (the state recurrence) and K4 (head
// RMSNorm, sigmoid output gate) fused in one kernel, one workgroup per (head, sequence).
//
// Replaces, for T = 1, the reference's k3_kda_layer body between the projections and o_proj
// (src/core/k3_ops.c:896-947): k3_shortconv + SiLU (:133-165), l2norm_ (:845-851), beta
// (:903), k3_kda_decay (:168-183), k3_kda_step (:186-243), k3_rmsnorm (:94-102) and the
// sigmoid gate (:940-947).
//
// Everything a (head, sequence) pair needs is local to it: its rows of the projections,
// its conv history and its D x D state. Fusing the three stages keeps q, k, v, alpha, beta
// and o in LDS instead of HBM and removes two launches per layer step; the state read is
// issued first so its HBM latency overlaps the K1 arithmetic. A batch's states larger than
// STATE_CACHED_BYTES stream through with nontemporal loads and stores (not kept in the
// caches): the batch-16 decode layer at hidden 7168 measured 97.5 -> 91 us with them. Smaller
// ones (a batch-1 decode: 2 MiB at H=32, D=128) use ordinary loads and stores, so the next
// token's launch finds its head's state in the L2 of the XCD the head runs on (workgroup
// (h, b) is dispatched to the same XCD every launch).
//
// Arithmetic: K1 is that of kda_prep_math.h with one half-wave per row (the wide prep
// kernel's layout: CPL = max(1, D/32) adjacent channels per lane, fp32 L2 sums), K3 that of
// kda_decode_kernel (same thread tile, same reduction order), K4 that of
// kda_epilogue2_kernel except for the row's sum of squares: fp32 per-lane squares added
// across the half-wave by DPP in fp32 (the epilogue kernel adds the lanes in double; for a
// 128-channel head the two differ by a few 1e-7 relative) and the hardware reciprocal
// square root; hardware sigmoid. The output-gate logits may arrive as split-K partial planes of the gate
// projection; they are added in plane order, which is what the split-K reduction does.
//
// The core form (k3hip_kda_decode_step) takes the decay logits z and the conv inputs as
// arrays of their own (bf16 or fp32), the output-gate logits as one array (bf16 or fp32) and
// writes y in fp32 or bf16; the state S and the conv history may live in separate arrays.
// It is one launch per decode token for K1 (T = 1) + K3 + K4, the work of k3hip_kda_prep,
// k3hip_kda_decode and k3hip_kda_epilogue in three.
//
// In the layer form, the decay logits z = f_a . W_fb^T (the f_b projection, k3_ops.c:886, D
// outputs of the head from the D-wide f_a row) are computed here too, one 16-channel group of W_fb per
// wave, in the arithmetic of the decode GEMV (kda_rows.hip): f_a split into bf16 hi + lo
// against the bf16 weight fragments, each 32-wide K-step's product an fp32 partial of its
// own, the partials added in K-step order. z gets the bits the stand-alone GEMV gives it,
// without its launch and its round trip through memory (batch-16 decode layer at hidden
// 7168: one launch of ~5 us fewer per layer).
#include "kda_internal.h"
#include "kda_prep_math.h"
#include "kda_split.h"

namespace k3kda {

constexpr size_t STATE_CACHED_BYTES = 8u << 20;

// Where the step kernel finds its operands for sequence b (row strides in elements).
struct StepArgs {
    int H;
    float lb, eps, q_scale;
    const void *qi, *ki, *vi;   // conv inputs, row b at b * ldi, in_dt storage
    long ldi;
    int in_dt;
    const float *bl;            // beta logits, row b at b * ldb (H of them)
    long ldb;
    const float *fa;            // layer form: f_a row b at b * ldfa (D wide) ...
    long ldfa;
    const uint16_t *Wfb;        // ... against W_fb in fragment order
    const float *z;             // core form: decay logits row b at b * ldz (P wide)
    long ldz;
    const void *gl;             // output-gate logits [B][P] (g_dt), or gsplit fp32 planes
    int g_dt, gsplit;
    long gplane;
    const float *q_conv, *k_conv, *v_conv, *A_log, *dt_bias, *o_norm;
    float *S;                   // sequence b's H x D x D state at b * s_stride
    long s_stride;
    float *hist;                // sequence b's [3][P][K-1] conv history at b * h_stride
    long h_stride;
    void *y;                    // [B][P], y_dt
    int y_dt;
    float *zout;                // zn floats zeroed on the way (may be nullptr)
    long zn;
    int stream_state;           // 1: nontemporal state loads and stores
};

template <int D, int K, bool ZIN>
__global__ __launch_bounds__(4 * D) void kda_layer_step_kernel(const StepArgs a)
{
#pragma clang fp contract(off)
    constexpr int NT = 4 * D;
    constexpr int CPR = D / 4;      // float4 column groups per state row
    constexpr int RPP = NT / CPR;   // rows covered by one pass of the workgroup (16)
    constexpr int NPASS = D / RPP;  // float4s of state held per thread
    static_assert(CPR * RPP == NT && NPASS * RPP == D, "tile shape");
    constexpr int CPL = D >= 32 ? D / 32 : 1;   // K1 channels per lane of a half-wave
    constexpr int NH = K - 1;
    constexpr int HWS = NT / 32;                // half-waves
    constexpr int TPT = (4 + HWS - 1) / HWS;    // K1 tasks per half-wave

    __shared__ float s_q[D], s_k[D], s_v[D], s_a[D], s_z[D];
    __shared__ f4 s_upart[RPP][CPR];   // per row slot and column group: partial u = S^T k
    __shared__ f4 s_opart[RPP][CPR];   // the same for o = S^T q
    __shared__ float s_beta;

    const int H = a.H;
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int cg = tid % CPR, rs = tid / CPR;
    const size_t P = (size_t)H * D;

    // Core form: every global operand is requested up front, so the step waits for memory
    // once: this thread's K1 inputs (task hw + i HWS: 0..2 = q, k, v conv, 3 = the decay
    // gate), the state, the beta logit and, for the K4 lanes, the gate logits and o_norm. The
    // layer form loads its K1 and K4 operands where it uses them: holding them across the
    // z product would take its registers from 90 to 152 and halve the workgroups per CU
    // (batch-16 step 16 -> 20 us).
    const int hw = tid >> 5, l32 = tid & 31;
    const bool active = l32 * CPL < D;
    const int cl = active ? l32 * CPL : 0;   // channel within the head
    const size_t c0 = (size_t)h * D + cl;
    float *hist = a.hist + (size_t)b * a.h_stride;   // [3][P][K-1]
    float pcur[TPT][CPL], pw[TPT][CPL][K], ph[TPT][CPL][NH > 0 ? NH : 1], pz[CPL], pdt[CPL];
    float pA = 0.0f;
    auto k1_operands = [&](int i) {
        const int task = hw + i * HWS;
        if (task < 3) {
            const float *cw = task == 0 ? a.q_conv : (task == 1 ? a.k_conv : a.v_conv);
            const void *src = task == 0 ? a.qi : (task == 1 ? a.ki : a.vi);
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const size_t ch = c0 + e;
                const size_t at = (size_t)b * a.ldi + ch;
                pcur[i][e] = a.in_dt == K3HIP_BF16 ? load_act<K3HIP_BF16>(src, at) : load_act<K3HIP_F32>(src, at);
#pragma unroll
                for (int j = 0; j < K; j++) pw[i][e][j] = cw[ch * K + j];
                const float *hs = hist + ((size_t)task * P + ch) * NH;
#pragma unroll
                for (int j = 0; j < NH; j++) ph[i][e][j] = hs[j];
            }
        } else if (task == 3) {
            pA = a.A_log[h];
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                pdt[e] = a.dt_bias[c0 + e];
                if constexpr (ZIN) pz[e] = a.z[(size_t)b * a.ldz + c0 + e];
            }
        }
    };
    const size_t at4 = (size_t)b * P + (size_t)h * D + 4 * (tid % CPR);
    f4 gt = 0.0f, wn = 0.0f;
    auto k4_operands = [&]() {
        if (tid >= CPR) return;
        if (a.g_dt == K3HIP_BF16) {
            const uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.gl) + at4);
            gt = f4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                    __uint_as_float(v.y & 0xffff0000u)};
        } else {
            const float *g32 = reinterpret_cast<const float *>(a.gl);
            gt = *reinterpret_cast<const f4 *>(g32 + at4);
            for (int sp = 1; sp < a.gsplit; sp++)
                gt = gt + *reinterpret_cast<const f4 *>(g32 + (size_t)sp * a.gplane + at4);
        }
        wn = reinterpret_cast<const f4 *>(a.o_norm)[tid];
    };
    if constexpr (ZIN) {
#pragma unroll
        for (int i = 0; i < TPT; i++) k1_operands(i);
        k4_operands();
    }
    float pbl = 0.0f;
    if (tid == 0) pbl = a.bl[(size_t)b * a.ldb + h];

    // layer form, z: wave wv takes the head's 16-channel group wv of W_fb (D / 16 groups =
    // NT / 64 waves); A-operand row 0 is this sequence's f_a, rows 1..15 zero.
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int KT = (D + 31) / 32;   // K-steps over the D-wide f_a
    const int ln = tid & 63, r16 = ln & 15, kq = ln >> 4, wv = tid >> 6;
    bsplit::bf16x8 wfr[KT];
    f4 fxa[KT], fxb[KT];
    if constexpr (!ZIN) {
        const bsplit::bf16x8 *wf = reinterpret_cast<const bsplit::bf16x8 *>(a.Wfb) +
                                   ((size_t)h * (D / 16) + wv) * KT * 64 + ln;
        const float *fa = a.fa + (size_t)b * a.ldfa;
#pragma unroll
        for (int t = 0; t < KT; t++) {
            wfr[t] = wf[(size_t)t * 64];
            const int k = 32 * t + 8 * kq;   // D % 8 == 0: the 8-slice is wholly inside or outside
            fxa[t] = fxb[t] = f4(0.0f);
            if (r16 == 0 && k < D) {
                fxa[t] = f4{fa[k], fa[k + 1], fa[k + 2], fa[k + 3]};
                fxb[t] = f4{fa[k + 4], fa[k + 5], fa[k + 6], fa[k + 7]};
            }
        }
    }

    // the state
    f4 *Sp = reinterpret_cast<f4 *>(a.S + (size_t)b * a.s_stride + (size_t)h * D * D);
    f4 s[NPASS];
#pragma unroll
    for (int m = 0; m < NPASS; m++)
        s[m] = a.stream_state ? __builtin_nontemporal_load(&Sp[(rs + m * RPP) * CPR + cg]) : Sp[(rs + m * RPP) * CPR + cg];

    // zout[0 .. zn) = 0 for the o_proj product that adds its two K-range partials there
    // (stream-ordered after every reader of the layer input), spread over the grid
    if (a.zout) {
        const long nwg = (long)gridDim.x * gridDim.y, id = (long)b * gridDim.x + h;
        const long per = (a.zn + nwg - 1) / nwg, z0 = id * per, z1 = min(a.zn, z0 + per);
        for (long i = z0 + tid; i < z1; i += NT) a.zout[i] = 0.0f;
    }

    if constexpr (!ZIN) {
        f32x4 zs = 0.0f;
#pragma unroll
        for (int t = 0; t < KT; t++) {
            bsplit::bf16x8 xh, xl;
            bsplit::split_row8(fxa[t], fxb[t], xh, xl);
            f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wfr[t], f32x4(0.0f), 0, 0, 0);
            p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wfr[t], p, 0, 0, 0);
            zs = t == 0 ? p : zs + p;
        }
        if (ln < 16) s_z[16 * wv + ln] = zs[0];   // C layout: lane n < 16 holds row 0, column n
        __syncthreads();
#pragma unroll
        for (int e = 0; e < CPL; e++) pz[e] = s_z[cl + e];
    }

    // K1
#pragma unroll
    for (int i = 0; i < TPT; i++) {
        const int task = hw + i * HWS;
        if constexpr (!ZIN) k1_operands(i);
        if (task < 3) {
            float yv[CPL];
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const size_t ch = c0 + e;
                yv[e] = active ? conv_silu<K>(pw[i][e], ph[i][e], pcur[i][e]) : 0.0f;
                if (active) {
                    float *hs = hist + ((size_t)task * P + ch) * NH;
#pragma unroll
                    for (int j = 0; j + 1 < NH; j++) hs[j] = ph[i][e][j + 1];
                    if constexpr (NH > 0) hs[NH - 1] = pcur[i][e];
                }
            }
            if (task < 2) l2norm_half<CPL>(yv);   // uniform per half-wave: both halves of a wave
            float *dst = task == 0 ? s_q : (task == 1 ? s_k : s_v);
            if (active)
#pragma unroll
                for (int e = 0; e < CPL; e++) dst[cl + e] = task == 0 ? yv[e] * a.q_scale : yv[e];
        } else if (task == 3 && active) {
            const float ea = expf(pA);
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const float g = a.lb != 0.0f ? gate_bounded(a.lb, gate_a2(ea), pz[e], pdt[e])
                                             : -ea * softplus_ref(pz[e] + pdt[e]);   // softplus gate
                s_a[cl + e] = fast_exp(g);
            }
        }
    }
    if (tid == 0) s_beta = fast_sigmoid(pbl);
    __syncthreads();

    // K3 (kda_decode_kernel): decay the rows, partial u over this thread's rows
    const f4 vv = reinterpret_cast<const f4 *>(s_v)[cg];
    const float bt = s_beta;
    f4 u = 0.0f;
#pragma unroll
    for (int m = 0; m < NPASS; m++) {
        const int r = rs + m * RPP;
        const float kr = s_k[r];
        s[m] = s[m] * s_a[r];
        if (kr != 0.0f) u = u + kr * s[m];
    }
    // every thread adds its column group's RPP partials itself, in row-slot order (the same
    // bits as one reducing thread per group; no second barrier and no LDS round trip of u:
    // B=1, H=32 decode tail 5.59 -> 5.42 us per token); o's partials go to their own array,
    // so no barrier separates these reads from its writes
    s_upart[rs][cg] = u;
    __syncthreads();
    f4 ut = s_upart[0][cg];
#pragma unroll
    for (int r = 1; r < RPP; r++) ut = ut + s_upart[r][cg];
    const f4 d = vv - ut;
    f4 acc = 0.0f;
#pragma unroll
    for (int m = 0; m < NPASS; m++) {
        const int r = rs + m * RPP;
        const float kr = s_k[r], qr = s_q[r];
        if (kr != 0.0f) s[m] = s[m] + (kr * bt) * d;
        if (qr != 0.0f) acc = acc + qr * s[m];
    }
    s_opart[rs][cg] = acc;
    if constexpr (!ZIN) k4_operands();
    __syncthreads();

    // K4 (kda_epilogue2_kernel's RMSNorm and gate) on o = the first CPR lanes' float4s, in the
    // first half-wave; the other waves store their part of the new state meanwhile (the
    // state stores, 4 D^2 bytes through one CU, take longer than K4)
    if (tid < 32) {
        f4 x = s_opart[0][tid < CPR ? tid : 0];
#pragma unroll
        for (int r = 1; r < RPP; r++) x = x + s_opart[r][tid < CPR ? tid : 0];
        const float part = tid < CPR ? ((x.x * x.x) + (x.y * x.y)) + ((x.z * x.z) + (x.w * x.w)) : 0.0f;
        const float inv = __builtin_amdgcn_rsqf(half_wave_sum(part) / (float)D + a.eps);
        if (tid < CPR) {
            f4 out;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gt[e] * 1.4426950408889634f));
                out[e] = ((wn[e] * x[e]) * inv) * sg;
            }
            if (a.y_dt == K3HIP_BF16) {
                const uint2 v = {(uint32_t)f2bf(out[0]) | ((uint32_t)f2bf(out[1]) << 16),
                                 (uint32_t)f2bf(out[2]) | ((uint32_t)f2bf(out[3]) << 16)};
                *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(a.y) + at4) = v;
            } else {
                *reinterpret_cast<f4 *>(reinterpret_cast<float *>(a.y) + at4) = out;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < NPASS; m++) {
        if (a.stream_state) __builtin_nontemporal_store(s[m], &Sp[(rs + m * RPP) * CPR + cg]);
        else Sp[(rs + m * RPP) * CPR + cg] = s[m];
    }
}

template <int D, bool ZIN>
static int launch_step(int K, int B, const StepArgs &a, hipStream_t st)
{
#define K3_STEP(KK) hipLaunchKernelGGL((kda_layer_step_kernel<D, KK, ZIN>), dim3(a.H, B), dim3(4 * D), 0, st, a)
    switch (K) {
    case 1: K3_STEP(1); break;
    case 2: K3_STEP(2); break;
    case 3: K3_STEP(3); break;
    case 4: K3_STEP(4); break;
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "decode step: conv_k=%d not in 1..4", K);
    }
#undef K3_STEP
    K3_LAUNCHED();
    return K3HIP_OK;
}

template <bool ZIN>
static int launch_step_d(int D, int K, int B, const StepArgs &a, hipStream_t st)
{
    switch (D) {
    case 16: return launch_step<16, ZIN>(K, B, a, st);
    case 32: return launch_step<32, ZIN>(K, B, a, st);
    case 64: return launch_step<64, ZIN>(K, B, a, st);
    case 128: return launch_step<128, ZIN>(K, B, a, st);
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "decode step: D=%d not in {16,32,64,128}", D);
    }
}

int layer_step(int B, int H, int D, int K, float lb, float eps, float q_scale, const float *Cin,
               long ldc, int bcol, int facol, const uint16_t *Wfb, const float *gl, int gsplit, long gplane,
               const float *q_conv, const float *k_conv, const float *v_conv, const float *A_log,
               const float *dt_bias, const float *o_norm, float *states, long stride, float *y,
               float *zout, long zn, hipStream_t st)
{
    if (B <= 0 || H <= 0) return K3HIP_OK;
    if (gsplit < 1 || ((uintptr_t)gl & 15) || (gplane & 3) || ((uintptr_t)y & 15) || ((uintptr_t)states & 15) ||
        (stride & 3) || ((uintptr_t)Wfb & 15) || (D & 7))
        K3_FAIL(K3HIP_EINVAL, "layer step: gate planes, y, states or W_fb misaligned");
    const size_t P = (size_t)H * D;
    StepArgs a{};
    a.H = H; a.lb = lb; a.eps = eps; a.q_scale = q_scale;
    a.qi = Cin; a.ki = Cin + P; a.vi = Cin + 2 * P; a.ldi = ldc; a.in_dt = K3HIP_F32;
    a.bl = Cin + bcol; a.ldb = ldc;
    a.fa = Cin + facol; a.ldfa = ldc; a.Wfb = Wfb;
    a.gl = gl; a.g_dt = K3HIP_F32; a.gsplit = gsplit; a.gplane = gplane;
    a.q_conv = q_conv; a.k_conv = k_conv; a.v_conv = v_conv; a.A_log = A_log; a.dt_bias = dt_bias; a.o_norm = o_norm;
    a.S = states; a.s_stride = stride; a.hist = states + P * D; a.h_stride = stride;
    a.y = y; a.y_dt = K3HIP_F32;
    a.zout = zout; a.zn = zn;
    a.stream_state = (size_t)B * P * D * 4 > STATE_CACHED_BYTES;
    return launch_step_d<false>(D, K, B, a, st);
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_kda_decode_step(int B, int H, int D, int K, float gate_lb, float rms_eps, int in_dtype,
                                     const void *q_in, const void *k_in, const void *v_in, const float *z,
                                     const float *b_logit, const void *gate, int gate_dtype,
                                     const float *q_conv, const float *k_conv, const float *v_conv,
                                     const float *A_log, const float *dt_bias, const float *o_norm,
                                     float *conv_state, float q_scale, float *S, void *y, int y_dtype,
                                     void *stream)
{
    clear_error();
    if (B < 0 || H <= 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode_step: B=%d H=%d", B, H);
    if (B == 0) return K3HIP_OK;
    if (!is_pow2_head(D)) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_decode_step: D=%d not in {16,32,64,128}", D);
    if (K < 1 || K > 4) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_decode_step: conv_k=%d not in 1..4", K);
    if (!(gate_lb <= 0.0f))
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode_step: gate_lb=%g (a bound <= 0; 0 selects the softplus gate)", gate_lb);
    if ((in_dtype != K3HIP_F32 && in_dtype != K3HIP_BF16) || (gate_dtype != K3HIP_F32 && gate_dtype != K3HIP_BF16) ||
        (y_dtype != K3HIP_F32 && y_dtype != K3HIP_BF16))
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode_step: dtypes in=%d gate=%d y=%d", in_dtype, gate_dtype, y_dtype);
    if (!q_in || !k_in || !v_in || !z || !b_logit || !gate || !q_conv || !k_conv || !v_conv || !A_log ||
        !dt_bias || !o_norm || !S || !y || (K > 1 && !conv_state))
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode_step: NULL argument (conv_state is needed for conv_k > 1)");
    const size_t P = (size_t)H * D;
    const uintptr_t ga = gate_dtype == K3HIP_F32 ? 15 : 7, ya = y_dtype == K3HIP_F32 ? 15 : 7;
    if ((((uintptr_t)S | (uintptr_t)o_norm) & 15) || ((uintptr_t)gate & ga) || ((uintptr_t)y & ya))
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode_step: S and o_norm need 16-byte alignment, gate and y 16 (fp32) "
                "or 8 (bf16)");
    StepArgs a{};
    a.H = H; a.lb = gate_lb; a.eps = rms_eps; a.q_scale = q_scale;
    a.qi = q_in; a.ki = k_in; a.vi = v_in; a.ldi = (long)P; a.in_dt = in_dtype;
    a.bl = b_logit; a.ldb = H;
    a.z = z; a.ldz = (long)P;
    a.gl = gate; a.g_dt = gate_dtype; a.gsplit = 1; a.gplane = 0;
    a.q_conv = q_conv; a.k_conv = k_conv; a.v_conv = v_conv; a.A_log = A_log; a.dt_bias = dt_bias; a.o_norm = o_norm;
    a.S = S; a.s_stride = (long)(P * D);
    a.hist = conv_state; a.h_stride = (long)(3 * P * (size_t)(K - 1));
    a.y = y; a.y_dt = y_dtype;
    a.stream_state = (size_t)B * P * D * 4 > STATE_CACHED_BYTES;
    return launch_step_d<true>(D, K, B, a, as_stream(stream));
}
