/*
 * Runs the oracle (oracle/gtmoe_oracle.c, included whole) under
 * AddressSanitizer and UndefinedBehaviorSanitizer on small mixtures of
 * experts: every precision, shared experts, clamped SwiGLU, hash routing,
 * learned routing with ties and NaN logits, widths off the 16-value blocks,
 * one and several threads, the stack and its routed form.  Checks the
 * reference invariants on the way (k distinct experts per token, gates
 * summing to 1, loads summing to T*k, threads not changing results, the
 * routed forward equal to the full one).  Exits 0 when every check held.
 */
#include "gtmoe_oracle.c"

#include <stdio.h>

static int failures = 0;
#define CHECK(cond, msg)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            fprintf(stderr, "FAILED: %s (line %d)\n", msg, __LINE__); \
            ++failures;                                    \
        }                                                  \
    } while (0)

static uint64_t rng_state = 0x9e3779b97f4a7c15ULL;
static double uniform(void)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (double)(rng_state >> 11) / 9007199254740992.0 * 2.0 - 1.0;
}

typedef struct {
    float *f32;
    int8_t *i8;
    uint8_t *fp4;
    float *scales;
    double *bias;
} storage;

static gtmoe_oracle_layer make_layer(int precision, int rows, int width, int activation, double limit, storage *s)
{
    size_t n = (size_t)rows * width;
    double *v = malloc(sizeof(double) * n);
    for (size_t i = 0; i < n; i++) v[i] = 0.3 * uniform();
    int blocks = scale_blocks(width);
    s->f32 = malloc(sizeof(float) * n + 4);
    s->i8 = malloc(n + 1);
    s->fp4 = malloc((size_t)rows * fp4_row_bytes(width) + 1);
    s->scales = malloc(sizeof(float) * (size_t)rows * blocks + 4);
    s->bias = malloc(sizeof(double) * (size_t)rows);
    for (int r = 0; r < rows; r++) s->bias[r] = 0.05 * uniform();
    gtmoe_oracle_encode_rows(precision, rows, width, v, s->f32, s->i8, s->fp4, s->scales);
    free(v);
    gtmoe_oracle_layer l;
    memset(&l, 0, sizeof l);
    l.weights.precision = precision;
    l.weights.rows = rows;
    l.weights.width = width;
    l.weights.values = precision == PREC_FLOAT32 ? (const void *)s->f32
                       : precision == PREC_INT8  ? (const void *)s->i8
                                                 : (const void *)s->fp4;
    l.weights.scales = s->scales;
    l.biases = s->bias;
    l.activation = activation;
    l.clamp_limit = limit;
    return l;
}

static void free_storage(storage *s)
{
    free(s->f32);
    free(s->i8);
    free(s->fp4);
    free(s->scales);
    free(s->bias);
}

static void run_case(int precision, int d, int h, int E, int k, int S, int hash, double clamp, int T)
{
    int G = S + E;
    storage *st = calloc((size_t)G * 3 + 1, sizeof(storage));
    gtmoe_oracle_expert *experts = calloc((size_t)G, sizeof(gtmoe_oracle_expert));
    for (int g = 0; g < G; g++) {
        experts[g].gate = make_layer(precision, h, d, clamp > 0 ? ACT_CLAMPED_SILU : ACT_SILU, clamp, &st[3 * g]);
        experts[g].up = make_layer(precision, h, d, clamp > 0 ? ACT_CLAMPED_LINEAR : ACT_LINEAR, clamp, &st[3 * g + 1]);
        experts[g].down = make_layer(precision, d, h, ACT_LINEAR, 0, &st[3 * g + 2]);
    }
    storage rs;
    double *balance = calloc((size_t)E, sizeof(double));
    gtmoe_oracle_moe moe;
    memset(&moe, 0, sizeof moe);
    moe.vector_size = d;
    moe.hidden_size = h;
    moe.shared_experts = S;
    moe.routed_experts = E;
    moe.experts_per_token = k;
    moe.use_hash_routing = hash;
    moe.shared = experts;
    moe.routed = experts + S;
    moe.router = make_layer(PREC_FLOAT32, E, d, ACT_LINEAR, 0, &rs);
    moe.balance_biases = balance;

    double *x = malloc(sizeof(double) * (size_t)T * d);
    for (int i = 0; i < T * d; i++) x[i] = uniform();
    int64_t *ids = malloc(sizeof(int64_t) * (size_t)T);
    for (int t = 0; t < T; t++) ids[t] = (int64_t)t * 7919 + 3;
    double *y1 = malloc(sizeof(double) * (size_t)T * d), *y3 = malloc(sizeof(double) * (size_t)T * d);
    double *yr = malloc(sizeof(double) * (size_t)T * d);
    int32_t *chosen = malloc(sizeof(int32_t) * (size_t)T * k), *load = malloc(sizeof(int32_t) * (size_t)E);
    double *gates = malloc(sizeof(double) * (size_t)T * k);
    CHECK(gtmoe_oracle_moe_forward(&moe, T, x, ids, 1, y1, chosen, gates, load, NULL, NULL) == 0, "forward");
    CHECK(gtmoe_oracle_moe_forward(&moe, T, x, ids, 3, y3, NULL, NULL, NULL, NULL, NULL) == 0, "forward 3 threads");
    CHECK(memcmp(y1, y3, sizeof(double) * (size_t)T * d) == 0, "threads changed the result");
    long total = 0;
    for (int e = 0; e < E; e++) total += load[e];
    CHECK(total == (long)T * k, "loads do not sum to T*k");
    for (int t = 0; t < T; t++) {
        double sum = 0;
        for (int i = 0; i < k; i++) {
            sum += gates[t * k + i];
            for (int j = 0; j < i; j++) CHECK(chosen[t * k + i] != chosen[t * k + j], "an expert chosen twice");
            CHECK(chosen[t * k + i] >= 0 && chosen[t * k + i] < E, "expert index out of range");
        }
        CHECK(fabs(sum - 1) <= 1e-12, "gates do not sum to 1");
    }
    gtmoe_oracle_moe_forward_routed(&moe, T, x, chosen, gates, 2, yr, NULL);
    CHECK(memcmp(y1, yr, sizeof(double) * (size_t)T * d) == 0, "routed forward differs");
    if (hash) {
        ids[0] = -1;
        CHECK(gtmoe_oracle_moe_forward(&moe, T, x, ids, 1, y1, NULL, NULL, NULL, NULL, NULL) == -1,
              "a negative id was taken");
    }

    /* the stack and its routed form over two copies of the layer */
    if (!hash) {
        gtmoe_oracle_moe layers[2] = {moe, moe};
        double *norm = malloc(sizeof(double) * (size_t)d);
        for (int i = 0; i < d; i++) norm[i] = 1 + 0.1 * uniform();
        const double *norms[2] = {norm, norm};
        double *xs = malloc(sizeof(double) * (size_t)T * d), *xr = malloc(sizeof(double) * (size_t)T * d);
        memcpy(xs, x, sizeof(double) * (size_t)T * d);
        memcpy(xr, x, sizeof(double) * (size_t)T * d);
        int32_t *sc = malloc(sizeof(int32_t) * 2 * (size_t)T * k);
        double *sg = malloc(sizeof(double) * 2 * (size_t)T * k);
        CHECK(gtmoe_oracle_stack_forward(layers, norms, 2, T, xs, NULL, 2, sc) == 0, "stack");
        /* gates of each layer from its own routing, for the routed form */
        double *xn = malloc(sizeof(double) * (size_t)T * d), *lg = malloc(sizeof(double) * (size_t)T * E);
        double *tmp = malloc(sizeof(double) * (size_t)T * d);
        memcpy(tmp, x, sizeof(double) * (size_t)T * d);
        for (int l = 0; l < 2; l++) {
            gtmoe_oracle_rmsnorm(T, d, tmp, norm, 1e-6, xn);
            gtmoe_oracle_layer_forward(&moe.router, T, xn, 1, lg);
            gtmoe_oracle_route_from_logits(T, E, k, lg, balance, sc + (size_t)l * T * k, sg + (size_t)l * T * k, NULL);
            gtmoe_oracle_moe_forward_routed(&moe, T, xn, sc + (size_t)l * T * k, sg + (size_t)l * T * k, 1, yr, NULL);
            for (int i = 0; i < T * d; i++) tmp[i] += yr[i];
        }
        gtmoe_oracle_stack_forward_routed(layers, norms, 2, T, xr, sc, sg, 1);
        CHECK(memcmp(xs, xr, sizeof(double) * (size_t)T * d) == 0, "routed stack differs");
        free(norm); free(xs); free(xr); free(sc); free(sg); free(xn); free(lg); free(tmp);
    }

    for (int i = 0; i < G * 3; i++) free_storage(&st[i]);
    free_storage(&rs);
    free(st); free(experts); free(balance); free(x); free(ids); free(y1); free(y3); free(yr);
    free(chosen); free(load); free(gates);
}

static void routing_edges(void)
{
    enum { T = 4, E = 6, K = 3 };
    double logits[T * E] = {
        0, 0, 0, 0, 0, 0,                                   /* all tied: lowest indices */
        NAN, 1, 2, NAN, 3, -1,                              /* NaN logits */
        25, -25, 19.9, 20.1, -19.9, -20.1,                  /* every softplus branch */
        INFINITY, -INFINITY, 1, 1, 1, 1,
    };
    double balance[E] = {0, 0.5, 0, -0.5, 0, 0};
    int32_t chosen[T * K];
    double gates[T * K], aff[T * E];
    int32_t load[E], offsets[E + 1], rows[T * K];
    gtmoe_oracle_route_from_logits(T, E, K, logits, balance, chosen, gates, aff);
    for (int i = 0; i < T * K; i++) CHECK(chosen[i] >= 0 && chosen[i] < E, "expert index out of range");
    CHECK(chosen[0] == 0 && chosen[1] == 1 && chosen[2] == 2, "ties keep the lower index");
    gtmoe_oracle_dispatch(T, E, K, chosen, load, offsets, rows);
    CHECK(offsets[E] == T * K, "dispatch offsets");
    int64_t ids[T] = {0, 1, (int64_t)1 << 40, 123456789};
    CHECK(gtmoe_oracle_hash_route(T, E, K, ids, chosen, gates) == 0, "hash route");
    double in[6] = {-745, -1e-300, 0, 1e-300, 709, 710}, out[6];
    for (int fn = 0; fn < 5; fn++) gtmoe_oracle_map(fn, 6, in, out);
}

int main(void)
{
    routing_edges();
    const int precisions[3] = {PREC_FLOAT32, PREC_INT8, PREC_FP4};
    for (int p = 0; p < 3; p++) {
        run_case(precisions[p], 20, 12, 5, 2, 1, 0, 0.0, 9);   /* widths off the 16-value blocks */
        run_case(precisions[p], 33, 17, 4, 4, 0, 0, 0.0, 5);   /* k = E */
        run_case(precisions[p], 16, 8, 6, 2, 2, 1, 0.0, 7);    /* hash routing, two shared */
        run_case(precisions[p], 48, 40, 8, 3, 1, 0, 0.7, 140); /* clamped, enough work to split threads */
    }
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("oracle_check: clean\n");
    return 0;
}
