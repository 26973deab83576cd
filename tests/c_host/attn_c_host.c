/*
 * A plain-C host of the attention ABI: what a non-Python caller (the Rust
 * CustomOp3 shim, a C++ trainer) does through include/foundry_attn.h.
 *
 * It allocates device buffers with the HIP runtime, runs fa_attn_fwd and
 * fa_attn_bwd on them, and checks O, LSE, dQ, dK, dV against the CPU oracle
 * (oracle/oracle.h, test infrastructure) on the same inputs, at the gates the
 * Python parity tests use: bf16 max-abs <= 2e-2 and rel-L2 <= 1e-2, LSE
 * max-abs <= 2e-3; f32 rel-L2 <= 1e-4.  It also checks the ABI's error
 * reporting.  Exit status 0 = every case passed.
 *
 * The reference runs the same op as q.apply_op3(&k, &v, AttnBwd)
 * (crates/foundry-spike/src/lib.rs:366) and AttnBwd::bwd (lib.rs:216-263).
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "foundry_attn.h"
#include "oracle.h"

static int failures = 0;

#define HIP_OK(call)                                                                  \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) {                                                       \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #call, hipGetErrorString(e_)); \
            exit(2);                                                                  \
        }                                                                             \
    } while (0)

static void expect(int ok, const char *what) {
    printf("  [%s] %s\n", ok ? "ok" : "FAIL", what);
    fflush(stdout);
    if (!ok) ++failures;
}

/* deterministic N(0,1) samples (xorshift + Box-Muller) */
static uint64_t rng_state = 20261028u;
static double uniform01(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return ((rng_state >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
static float normal01(void) {
    const double u = uniform01(), v = uniform01();
    return (float)(sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v));
}

static uint16_t to_bf16(float x) { /* round to nearest even; inputs are finite */
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static float from_bf16(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* max |a-b| and ||a-b|| / ||b|| over the elements of heads [h0, h1) of a
 * [B,S,H,D] array */
static void diff_heads(const float *a, const float *b, int B, int S, int H, int D, int h0, int h1,
                       double *max_abs, double *rel) {
    double num = 0, den = 0, mx = 0;
    for (long bs = 0; bs < (long)B * S; ++bs)
        for (int h = h0; h < h1; ++h)
            for (int d = 0; d < D; ++d) {
                const long i = (bs * H + h) * D + d;
                const double e = (double)a[i] - b[i];
                num += e * e;
                den += (double)b[i] * b[i];
                if (fabs(e) > mx) mx = fabs(e);
            }
    *max_abs = mx;
    *rel = den > 0 ? sqrt(num / den) : sqrt(num);
}

/* One fwd+bwd through the ABI, checked on heads [h0, h1). */
static void run_case(const char *name, int dtype, int B, int S, int H, int D, int masked, int h0, int h1) {
    const int bf = dtype == FA_DTYPE_BF16;
    const long n = (long)B * S * H * D;
    const size_t esz = bf ? 2 : 4;
    printf("%s: %s B=%d S=%d H=%d D=%d%s\n", name, bf ? "bf16" : "f32", B, S, H, D, masked ? " key mask" : "");
    fflush(stdout);

    float *host[4];
    for (int t = 0; t < 4; ++t) {
        host[t] = (float *)malloc(n * sizeof(float));
        for (long i = 0; i < n; ++i) host[t][i] = normal01();
        if (bf) oracle_round_bf16_inplace(host[t], n);
    }
    uint8_t *keep = NULL;
    if (masked) {
        keep = (uint8_t *)malloc((size_t)B * S);
        for (long i = 0; i < (long)B * S; ++i) keep[i] = uniform01() > 0.2;
        for (int b = 0; b < B; ++b) keep[(long)b * S] = 1;
    }
    const float scale = 1.0f / sqrtf((float)D);

    /* device buffers: q, k, v, dout, o, dq, dk, dv; lse; mask */
    void *dev[8];
    void *stage = malloc(n * esz);
    for (int t = 0; t < 8; ++t) HIP_OK(hipMalloc(&dev[t], n * esz));
    for (int t = 0; t < 4; ++t) {
        if (bf)
            for (long i = 0; i < n; ++i) ((uint16_t *)stage)[i] = to_bf16(host[t][i]);
        else
            memcpy(stage, host[t], n * 4);
        HIP_OK(hipMemcpy(dev[t], stage, n * esz, hipMemcpyHostToDevice));
    }
    float *dlse;
    HIP_OK(hipMalloc((void **)&dlse, (size_t)B * H * S * 4));
    uint8_t *dkeep = NULL;
    if (masked) {
        HIP_OK(hipMalloc((void **)&dkeep, (size_t)B * S));
        HIP_OK(hipMemcpy(dkeep, keep, (size_t)B * S, hipMemcpyHostToDevice));
    }
    const fa_strides st = {(int64_t)S * H * D, (int64_t)H * D, D};

    fa_attn_fwd_args fa;
    memset(&fa, 0, sizeof fa);
    fa.dtype = dtype;
    fa.batch = B;
    fa.seq = S;
    fa.heads = H;
    fa.head_dim = D;
    fa.scale = scale;
    fa.q = dev[0];
    fa.k = dev[1];
    fa.v = dev[2];
    fa.o = dev[4];
    fa.lse = dlse;
    fa.key_keep = dkeep;
    fa.q_stride = fa.k_stride = fa.v_stride = fa.o_stride = st;
    /* a grid too small for the GPU splits its keys when given the workspace
       the library asks for (0 = these shapes never split) */
    const size_t fws = fa_attn_fwd_workspace_size(&fa);
    if (fws > 0) {
        printf("  split forward: %zu workspace bytes\n", fws);
        HIP_OK(hipMalloc(&fa.workspace, fws));
        fa.workspace_bytes = fws - 256;
        expect(fa_attn_fwd(&fa, NULL) == FA_ERR_INVALID_ARG && fa_last_error()[0] != 0,
               "a forward workspace 256 bytes short is refused with a message");
        fa.workspace_bytes = fws;
    }
    expect(fa_attn_fwd(&fa, NULL) == FA_OK, "fa_attn_fwd returns FA_OK");

    fa_attn_bwd_args ba;
    memset(&ba, 0, sizeof ba);
    ba.dtype = dtype;
    ba.batch = B;
    ba.seq = S;
    ba.heads = H;
    ba.head_dim = D;
    ba.scale = scale;
    ba.q = dev[0];
    ba.k = dev[1];
    ba.v = dev[2];
    ba.o = dev[4];
    ba.dout = dev[3];
    ba.lse = dlse;
    ba.key_keep = dkeep;
    ba.dq = dev[5];
    ba.dk = dev[6];
    ba.dv = dev[7];
    ba.q_stride = ba.k_stride = ba.v_stride = ba.o_stride = ba.do_stride = st;
    ba.dq_stride = ba.dk_stride = ba.dv_stride = st;
    const size_t ws_bytes = fa_attn_bwd_workspace_size(&ba);
    const size_t ws_min = fa_attn_bwd_min_workspace_size(&ba);
    expect(ws_bytes > 0 && ws_min > 0 && ws_min <= ws_bytes,
           "fa_attn_bwd_workspace_size >= fa_attn_bwd_min_workspace_size > 0");
    ba.workspace_bytes = ws_min - 1;
    HIP_OK(hipMalloc(&ba.workspace, ws_bytes));
    expect(fa_attn_bwd(&ba, NULL) == FA_ERR_INVALID_ARG && fa_last_error()[0] != 0,
           "a workspace one byte under the minimum is refused with a message");
    ba.workspace_bytes = ws_bytes;
    expect(fa_attn_bwd(&ba, NULL) == FA_OK, "fa_attn_bwd returns FA_OK");
    HIP_OK(hipDeviceSynchronize());

    /* device results -> f32 */
    float *got[4]; /* o, dq, dk, dv */
    const int order[4] = {4, 5, 6, 7};
    for (int t = 0; t < 4; ++t) {
        got[t] = (float *)malloc(n * sizeof(float));
        HIP_OK(hipMemcpy(stage, dev[order[t]], n * esz, hipMemcpyDeviceToHost));
        for (long i = 0; i < n; ++i) got[t][i] = bf ? from_bf16(((uint16_t *)stage)[i]) : ((float *)stage)[i];
    }
    float *glse = (float *)malloc((size_t)B * H * S * 4);
    HIP_OK(hipMemcpy(glse, dlse, (size_t)B * H * S * 4, hipMemcpyDeviceToHost));

    /* oracle on heads [h0, h1) */
    float *want[4], *wlse = (float *)calloc((size_t)B * H * S, 4);
    for (int t = 0; t < 4; ++t) want[t] = (float *)calloc(n, sizeof(float));
    expect(oracle_attn_fwd(host[0], host[1], host[2], want[0], wlse, B, S, H, D, scale, keep, bf, h0, h1, 0) == 0,
           "oracle forward");
    expect(oracle_attn_bwd(host[0], host[1], host[2], host[3], want[1], want[2], want[3], B, S, H, D, scale, keep,
                           bf, h0, h1, 0) == 0,
           "oracle backward");
    const char *names[4] = {"O", "dQ", "dK", "dV"};
    for (int t = 0; t < 4; ++t) {
        double ma, rl;
        diff_heads(got[t], want[t], B, S, H, D, h0, h1, &ma, &rl);
        char msg[160];
        const int ok = bf ? (ma <= 2e-2 && rl <= 1e-2) : rl <= 1e-4;
        snprintf(msg, sizeof msg, "%s: max_abs %.3e rel_l2 %.3e", names[t], ma, rl);
        expect(ok, msg);
    }
    double lmax = 0;
    for (int b = 0; b < B; ++b)
        for (int h = h0; h < h1; ++h)
            for (int s = 0; s < S; ++s) {
                const long i = ((long)b * H + h) * S + s;
                const double e = fabs((double)glse[i] - wlse[i]);
                if (e > lmax) lmax = e;
            }
    char msg[96];
    snprintf(msg, sizeof msg, "LSE: max_abs %.3e", lmax);
    expect(bf ? lmax <= 2e-3 : lmax <= 1e-4, msg);

    for (int t = 0; t < 8; ++t) HIP_OK(hipFree(dev[t]));
    HIP_OK(hipFree(dlse));
    HIP_OK(hipFree(ba.workspace));
    if (fa.workspace) HIP_OK(hipFree(fa.workspace));
    if (dkeep) HIP_OK(hipFree(dkeep));
    for (int t = 0; t < 4; ++t) {
        free(host[t]);
        free(got[t]);
        free(want[t]);
    }
    free(keep);
    free(stage);
    free(glse);
    free(wlse);
}

int main(void) {
    printf("foundry_attn ABI %d, op \"%s\"\n", fa_version(), fa_op_name());
    expect(fa_version() == FA_ABI_VERSION, "fa_version() == FA_ABI_VERSION");
    expect(strcmp(fa_op_name(), "foundry-attn-bwd") == 0, "fa_op_name() is the reference's op name");
    expect(fa_init(0) == FA_OK, "fa_init(0) on the gfx950 device");

    /* argument validation happens before any device work */
    fa_attn_fwd_args bad;
    memset(&bad, 0, sizeof bad);
    bad.dtype = FA_DTYPE_BF16;
    bad.batch = bad.seq = bad.heads = 1;
    bad.head_dim = 96;
    bad.scale = 0.1f;
    const fa_status s = fa_attn_fwd(&bad, NULL);
    expect((s == FA_ERR_INVALID_ARG || s == FA_ERR_UNSUPPORTED) && fa_last_error()[0] != 0,
           "head_dim 96 is refused with a message");
    expect(fa_attn_fwd(NULL, NULL) == FA_ERR_INVALID_ARG, "NULL args are refused");

    run_case("bf16, ragged S, masked", FA_DTYPE_BF16, 2, 333, 3, 128, 1, 0, 3);
    run_case("bf16, D=64", FA_DTYPE_BF16, 1, 200, 2, 64, 0, 0, 2);
    run_case("f32, config c1 shape", FA_DTYPE_F32, 1, 256, 4, 64, 0, 0, 4);
    run_case("bf16, 8-wave workgroups", FA_DTYPE_BF16, 1, 1400, 40, 128, 0, 38, 40);
    run_case("bf16, range split (few heads), masked", FA_DTYPE_BF16, 1, 2048, 2, 128, 1, 0, 2);

    printf("%s (%d failure%s)\n", failures ? "FAILED" : "PASSED", failures, failures == 1 ? "" : "s");
    return failures ? 1 : 0;
}
