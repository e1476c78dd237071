/*
 * CPU oracle for the fused-MoE hot path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker. Nothing in the tinyserve_amd package links, loads or calls it.
 *
 * Plain sequential C restatements of:
 *   oracle_align        - moe_align_block_size (reference tinykernels.py:1070-1190): buckets with
 *                          the remote bucket E for negative ids (tinykernels.py:1141), per-bucket
 *                          padding to block_m (1152), stable order inside a bucket (1166),
 *                          pad value numel (1186), expert_ids by searchsorted(right=True) with -1
 *                          for the remote bucket and the tail (1185-1188), total = padded end.
 *   oracle_route        - _moe_route_kernel (tinykernels.py:1535-1571): p = exp(l - max) in fp32,
 *                          top-k by repeated argmax with first-index ties (1559-1564), weights
 *                          p / sum(selected p) or p / sum(all p) (1566), ids via expert_map (1567).
 *   oracle_router_logits- the router Linear of SparseMoE (serve.py:1039, 1079) as an fp32-accumulated
 *                          dot product in the summation order the GPU router uses (below).
 *   oracle_expf         - the fp32 exponential the router uses (same algorithm as the GPU's).
 * The reductions whose order the reference leaves open (sum(p), the dot product, exp) are fixed
 * here to the order the GPU kernels use, so routing compares bit for bit:
 *   dot(x, g): lane j in [0,64) accumulates, with fmaf from +0, x[h]*g[h] for h = c*512 + j*8 + i,
 *   increasing (c, i), h < H; the 64 partials are combined by an XOR butterfly (distances
 *   32,16,8,4,2,1: v[l] <- v[l] + v[l^s]); sum(all p) uses the same butterfly over per-lane sums
 *   of p[j + 64q], increasing q.
 * Build with -ffp-contract=off (oracle/Makefile) so the compiler adds no fused operations.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float oracle_expf(float x) {
    if (!(x >= -86.0f)) return 0.0f;
    if (x > 88.0f) return INFINITY;
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.42860682030941723e-06f, r);
    float p = 1.98412698412698413e-04f;
    p = fmaf(p, r, 1.38888888888888889e-03f);
    p = fmaf(p, r, 8.33333333333333333e-03f);
    p = fmaf(p, r, 4.16666666666666667e-02f);
    p = fmaf(p, r, 1.66666666666666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

static float butterfly64(float v[64]) {
    float t[64];
    for (int s = 32; s >= 1; s >>= 1) {
        for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ s];
        memcpy(v, t, sizeof(t));
    }
    return v[0];
}

static float bf16_bits_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float round_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u = (u | 0x00400000u) & 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    memcpy(&f, &u, 4);
    return f;
}

/* dtype: 0 = fp32, 1 = bf16 (raw uint16 bits) */
static float load_elem(const void* p, int dtype, int64_t i) {
    return dtype == 1 ? bf16_bits_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

float oracle_dot_ordered(const void* x, const void* g, int dtype, int H) {
    float v[64];
    for (int j = 0; j < 64; ++j) {
        float acc = 0.0f;
        for (int c = 0; c * 512 < H; ++c)
            for (int i = 0; i < 8; ++i) {
                int h = c * 512 + j * 8 + i;
                if (h < H) acc = fmaf(load_elem(x, dtype, h), load_elem(g, dtype, h), acc);
            }
        v[j] = acc;
    }
    return butterfly64(v);
}

void oracle_router_logits(const void* x, const void* gw, int dtype, int64_t T, int H, int E,
                          const float* bias, int logits_bf16, float* logits) {
    const size_t esz = dtype == 1 ? 2 : 4;
    for (int64_t t = 0; t < T; ++t)
        for (int e = 0; e < E; ++e) {
            float l = oracle_dot_ordered((const char*)x + (size_t)t * H * esz,
                                         (const char*)gw + (size_t)e * H * esz, dtype, H);
            if (bias) l = l + bias[e];
            if (logits_bf16) l = round_bf16(l);
            logits[t * E + e] = l;
        }
}

void oracle_route(const float* logits, int64_t T, int E, int64_t ld, int top_k, int renorm,
                  const int64_t* expert_map, float* w, int32_t* ids) {
    float* p = (float*)malloc(sizeof(float) * E);
    for (int64_t t = 0; t < T; ++t) {
        const float* l = logits + t * ld;
        float m = -INFINITY;
        for (int e = 0; e < E; ++e) m = fmaxf(m, l[e]);
        for (int e = 0; e < E; ++e) p[e] = oracle_expf(l[e] - m);
        float lanes[64];
        for (int j = 0; j < 64; ++j) {
            float s = 0.0f;
            for (int e = j; e < E; e += 64) s = s + p[e];
            lanes[j] = s;
        }
        float all = butterfly64(lanes);
        float sel = 0.0f;
        float sv[64];
        int si[64];
        for (int s = 0; s < top_k; ++s) {
            int bi = -1;
            float bv = -INFINITY;
            for (int e = 0; e < E; ++e)
                if (bi < 0 || p[e] > bv) { bv = p[e]; bi = e; }
            sv[s] = bv;
            si[s] = bi;
            sel = sel + bv;
            p[bi] = -INFINITY;
        }
        float denom = renorm ? sel : all;
        for (int s = 0; s < top_k; ++s) {
            w[t * top_k + s] = sv[s] / denom;
            ids[t * top_k + s] = expert_map ? (int32_t)expert_map[si[s]] : si[s];
        }
    }
    free(p);
}

int64_t oracle_max_padded(int64_t numel, int E, int block_m) {
    int64_t nb = E + 1;
    return (numel + nb * (block_m - 1) + block_m - 1) / block_m * block_m;
}

/* sorted_ids: [max_padded], expert_ids: [max_padded / block_m], total: [1] */
void oracle_align(const int32_t* ids, int64_t numel, int E, int block_m, int32_t* sorted_ids,
                  int32_t* expert_ids, int32_t* total) {
    const int nb = E + 1;
    const int64_t mp = oracle_max_padded(numel, E, block_m);
    int64_t* cnt = (int64_t*)calloc(nb, sizeof(int64_t));
    int64_t* start = (int64_t*)calloc(nb + 1, sizeof(int64_t));
    int64_t* fill = (int64_t*)calloc(nb, sizeof(int64_t));
    for (int64_t a = 0; a < numel; ++a) {
        int b = (ids[a] >= 0 && ids[a] < E) ? ids[a] : E;
        cnt[b]++;
    }
    for (int b = 0; b < nb; ++b)
        start[b + 1] = start[b] + (cnt[b] + block_m - 1) / block_m * block_m;
    for (int64_t r = 0; r < mp; ++r) sorted_ids[r] = (int32_t)numel;
    for (int64_t a = 0; a < numel; ++a) {   /* ascending a: stable within each bucket */
        int b = (ids[a] >= 0 && ids[a] < E) ? ids[a] : E;
        sorted_ids[start[b] + fill[b]++] = (int32_t)a;
    }
    for (int64_t tl = 0; tl < mp / block_m; ++tl) {
        int64_t row = tl * block_m;
        int b = 0;                           /* first bucket whose padded end exceeds row */
        while (b < nb && start[b + 1] <= row) ++b;
        expert_ids[tl] = b < E ? b : -1;
    }
    total[0] = (int32_t)start[nb];
    free(cnt);
    free(start);
    free(fill);
}
