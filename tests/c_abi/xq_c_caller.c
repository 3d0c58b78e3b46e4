/*
 * A plain-C caller of the library's ABI (include/xq_attn.h): no Python, no
 * torch, only the HIP runtime for device memory. It runs one q8_0
 * flash-attention decode (2 sequences, 8 heads over 2 KV heads, D 128, 300
 * rows) and one gated-delta-net prefill (5 tokens, two snapshot slots) on the
 * GPU, once with the step kernel and once with the chunked form, and checks
 * each against the CPU oracle within the parity tolerance (2e-3 abs + 1e-2
 * rel). Exit status 0 when every check passes.
 *
 * Test infrastructure: it links the oracle (oracle/_build/libxqoracle.so) as
 * the result it compares with, as the Python tests do.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "xq_attn.h"
#include "xq_oracle.h"

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;

/* uniform in [-1, 1) from xorshift64 */
static float urand(void) {
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (float)((double)(g_rng >> 11) * (1.0 / 9007199254740992.0) * 2.0 - 1.0);
}

static int g_fail = 0;

#define HIP_OK(x)                                                                 \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            exit(2);                                                              \
        }                                                                         \
    } while (0)

static void* to_device(const void* host, size_t bytes) {
    void* d = NULL;
    HIP_OK(hipMalloc(&d, bytes));
    HIP_OK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
    return d;
}

static xq_tensor tensor(int type, const int64_t ne[4], const size_t nb[4], void* data) {
    xq_tensor t;
    memset(&t, 0, sizeof t);
    t.type = type;
    for (int i = 0; i < 4; ++i) {
        t.ne[i] = ne[i];
        t.nb[i] = nb[i];
    }
    t.data = data;
    return t;
}

/* max |got - want| over n floats, failing when one is outside the tolerance */
static double compare(const char* what, const float* got, const float* want, size_t n) {
    double worst = 0.0;
    size_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        const double d = fabs((double)got[i] - (double)want[i]);
        if (!(d <= 2e-3 + 1e-2 * fabs((double)want[i]))) ++bad;
        if (d > worst) worst = d;
    }
    printf("%s: max|gpu - oracle| = %.3e, %zu of %zu outside the tolerance\n", what, worst, bad, n);
    if (bad) g_fail = 1;
    return worst;
}

static void check_status(const char* what, xq_status st) {
    if (st != XQ_OK) {
        fprintf(stderr, "%s: status %d (%s)\n", what, (int)st, xq_last_error());
        exit(3);
    }
}

static void fa_decode(void) {
    enum { D = 128, H = 8, HKV = 2, L = 300, NQ = 1, B = 2 };
    const size_t rec = D / 32 * 34; /* q8_0 record */
    float* q = malloc(sizeof(float) * D * H * NQ * B);
    uint8_t* k = malloc(rec * L * HKV * B);
    uint8_t* v = malloc(rec * L * HKV * B);
    float* row = malloc(sizeof(float) * D);
    for (int i = 0; i < D * H * NQ * B; ++i) q[i] = urand();
    for (int r = 0; r < L * HKV * B; ++r) {
        for (int i = 0; i < D; ++i) row[i] = urand();
        xo_quantize_row_q8_0(row, k + r * rec, D, 0);
        for (int i = 0; i < D; ++i) row[i] = urand();
        xo_quantize_row_q8_0(row, v + r * rec, D, 0);
    }
    const int64_t ne_q[4] = {D, NQ, H, B}, ne_kv[4] = {D, L, HKV, B}, ne_o[4] = {D, H, NQ, B};
    const size_t nb_q[4] = {4, H * D * 4, D * 4, (size_t)NQ * H * D * 4};
    const size_t nb_kv[4] = {34, HKV * rec, rec, (size_t)L * HKV * rec};
    const size_t nb_o[4] = {4, D * 4, H * D * 4, (size_t)NQ * H * D * 4};
    const size_t out_n = (size_t)D * H * NQ * B;
    float* want = calloc(out_n, sizeof(float));
    float* got = calloc(out_n, sizeof(float));

    xq_fa_params p;
    memset(&p, 0, sizeof p);
    p.scale = 1.0f / sqrtf((float)D);
    p.qk_policy = XQ_FA_QK_CONSISTENT;
    p.split_mode = XQ_FA_SPLIT_AUTO;
    p.engine = XQ_FA_ENGINE_AUTO;

    xq_tensor hq = tensor(XQ_TYPE_F32, ne_q, nb_q, q), hk = tensor(XQ_TYPE_Q8_0, ne_kv, nb_kv, k),
              hv = tensor(XQ_TYPE_Q8_0, ne_kv, nb_kv, v), ho = tensor(XQ_TYPE_F32, ne_o, nb_o, want);
    if (xo_flash_attn_ext(&hq, &hk, &hv, NULL, NULL, &ho, NULL, p.scale, 0.0f, 0.0f, p.qk_policy, 1, 4) != 0) {
        fprintf(stderr, "oracle flash_attn_ext failed\n");
        exit(3);
    }

    xq_tensor dq = tensor(XQ_TYPE_F32, ne_q, nb_q, to_device(q, sizeof(float) * D * H * NQ * B));
    xq_tensor dk = tensor(XQ_TYPE_Q8_0, ne_kv, nb_kv, to_device(k, rec * L * HKV * B));
    xq_tensor dv = tensor(XQ_TYPE_Q8_0, ne_kv, nb_kv, to_device(v, rec * L * HKV * B));
    xq_tensor dd = tensor(XQ_TYPE_F32, ne_o, nb_o, NULL);
    HIP_OK(hipMalloc(&dd.data, out_n * sizeof(float)));
    if (!xq_supports_flash_attn_ext(&dq, &dk, &dv, NULL, NULL, &dd, &p)) {
        fprintf(stderr, "flash_attn_ext not supported for the decode shape\n");
        exit(3);
    }
    size_t ws_bytes = 0;
    check_status("flash_attn_ext_workspace", xq_flash_attn_ext_workspace(&dq, &dk, &dv, NULL, NULL, &dd, &p, &ws_bytes));
    void* ws = NULL;
    if (ws_bytes) HIP_OK(hipMalloc(&ws, ws_bytes));
    check_status("flash_attn_ext", xq_flash_attn_ext(&dq, &dk, &dv, NULL, NULL, &dd, NULL, &p, ws, ws_bytes, NULL));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(got, dd.data, out_n * sizeof(float), hipMemcpyDeviceToHost));
    compare("flash_attn_ext q8_0 decode", got, want, out_n);

    hipFree(ws);
    hipFree(dq.data);
    hipFree(dk.data);
    hipFree(dv.data);
    hipFree(dd.data);
    free(q), free(k), free(v), free(row), free(want), free(got);
}

static void gdn_prefill(int32_t mode, const char* what) {
    enum { T = 5, B = 1, SLOTS = 2 };
    const int rows = T + SLOTS * 128;
    const size_t nq = (size_t)128 * 16 * T * B, nv = (size_t)128 * 32 * T * B, ngb = (size_t)32 * T * B;
    const size_t ns = (size_t)128 * 128 * 32 * B, nd = (size_t)4096 * rows * B;
    float *q = malloc(4 * nq), *k = malloc(4 * nq), *v = malloc(4 * nv), *g = malloc(4 * ngb), *be = malloc(4 * ngb);
    float* s = malloc(4 * ns);
    float *want = calloc(nd, 4), *got = calloc(nd, 4);
    for (size_t r = 0; r < nq / 128; ++r) { /* L2-normalised q and k rows */
        double sq = 0.0, sk = 0.0;
        for (int i = 0; i < 128; ++i) {
            q[r * 128 + i] = urand();
            k[r * 128 + i] = urand();
            sq += (double)q[r * 128 + i] * q[r * 128 + i];
            sk += (double)k[r * 128 + i] * k[r * 128 + i];
        }
        for (int i = 0; i < 128; ++i) {
            q[r * 128 + i] = (float)(q[r * 128 + i] / sqrt(sq));
            k[r * 128 + i] = (float)(k[r * 128 + i] / sqrt(sk));
        }
    }
    for (size_t i = 0; i < nv; ++i) v[i] = urand();
    for (size_t i = 0; i < ngb; ++i) {
        g[i] = -log1pf(expf(urand()));          /* -softplus */
        be[i] = 1.0f / (1.0f + expf(-urand())); /* sigmoid */
    }
    for (size_t i = 0; i < ns; ++i) s[i] = 0.1f * urand();

    const int64_t ne_qk[4] = {128, 16, T, B}, ne_v[4] = {128, 32, T, B}, ne_gb[4] = {1, 32, T, B};
    const int64_t ne_s[4] = {128, 128, 32, B}, ne_d[4] = {4096, rows, B, 1};
    const size_t nb_qk[4] = {4, 512, 512 * 16, (size_t)512 * 16 * T};
    const size_t nb_v[4] = {4, 512, 512 * 32, (size_t)512 * 32 * T};
    const size_t nb_gb[4] = {4, 4, 128, (size_t)128 * T};
    const size_t nb_s[4] = {4, 512, 65536, (size_t)65536 * 32};
    const size_t nb_d[4] = {4, 16384, (size_t)16384 * rows, (size_t)16384 * rows * B};

    xq_tensor hq = tensor(XQ_TYPE_F32, ne_qk, nb_qk, q), hk = tensor(XQ_TYPE_F32, ne_qk, nb_qk, k),
              hv = tensor(XQ_TYPE_F32, ne_v, nb_v, v), hg = tensor(XQ_TYPE_F32, ne_gb, nb_gb, g),
              hb = tensor(XQ_TYPE_F32, ne_gb, nb_gb, be), hs = tensor(XQ_TYPE_F32, ne_s, nb_s, s),
              hd = tensor(XQ_TYPE_F32, ne_d, nb_d, want);
    if (xo_gated_delta_net(&hq, &hk, &hv, &hg, &hb, &hs, &hd, SLOTS, 4) != 0) {
        fprintf(stderr, "oracle gated_delta_net failed\n");
        exit(3);
    }

    xq_tensor dq = tensor(XQ_TYPE_F32, ne_qk, nb_qk, to_device(q, 4 * nq));
    xq_tensor dk = tensor(XQ_TYPE_F32, ne_qk, nb_qk, to_device(k, 4 * nq));
    xq_tensor dv = tensor(XQ_TYPE_F32, ne_v, nb_v, to_device(v, 4 * nv));
    xq_tensor dg = tensor(XQ_TYPE_F32, ne_gb, nb_gb, to_device(g, 4 * ngb));
    xq_tensor db = tensor(XQ_TYPE_F32, ne_gb, nb_gb, to_device(be, 4 * ngb));
    xq_tensor ds = tensor(XQ_TYPE_F32, ne_s, nb_s, to_device(s, 4 * ns));
    xq_tensor dd = tensor(XQ_TYPE_F32, ne_d, nb_d, to_device(got, 4 * nd)); /* zeros */
    if (!xq_supports_gated_delta_net(&dq, &dk, &dv, &dg, &db, &ds, &dd, SLOTS, 0)) {
        fprintf(stderr, "gated_delta_net not supported for the prefill shape\n");
        exit(3);
    }
    size_t ws_bytes = 0;
    check_status("gated_delta_net_workspace", xq_gated_delta_net_workspace(&dq, &dv, SLOTS, mode, &ws_bytes));
    void* ws = NULL;
    if (ws_bytes) HIP_OK(hipMalloc(&ws, ws_bytes));
    check_status("gated_delta_net", xq_gated_delta_net(&dq, &dk, &dv, &dg, &db, &ds, &dd, SLOTS, 0, mode, ws, ws_bytes, NULL));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(got, dd.data, 4 * nd, hipMemcpyDeviceToHost));
    compare(what, got, want, nd);

    hipFree(ws);
    hipFree(dq.data), hipFree(dk.data), hipFree(dv.data), hipFree(dg.data), hipFree(db.data);
    hipFree(ds.data), hipFree(dd.data);
    free(q), free(k), free(v), free(g), free(be), free(s), free(want), free(got);
}

int main(void) {
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n));
    if (n < 1) {
        fprintf(stderr, "no GPU\n");
        return 2;
    }
    printf("library ABI %d\n", (int)xq_abi_version());
    fa_decode();
    gdn_prefill(XQ_GDN_STEP, "gated_delta_net 5 tokens, 2 slots, step kernel");
    gdn_prefill(XQ_GDN_CHUNKED, "gated_delta_net 5 tokens, 2 slots, chunked form");
    printf(g_fail ? "FAILED\n" : "all checks passed\n");
    return g_fail;
}
