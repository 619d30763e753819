/*
 * gtmoe_oracle.c -- CPU restatement of GoTransformers' mixture-of-experts
 * forward path over lowprecision rows.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only to check or time against; the product library
 * never links, calls or falls back to it.
 *
 * Every function follows the reference in float64 with the reference's loop
 * order.  Build with -ffp-contract=off: the reference's default amd64 build
 * never fuses a multiply with an add.
 *
 * Parity pins (what checks each part; the tests hold them):
 *   encode (Rows.Append)    closed forms, FP4 known answer, byte counts, halfway
 *                           and clamp cases, error bounds
 *   decode / DotRow         DotRow == Row().v within 1e-9; numpy brute force
 *   layer / SwiGLU / MoE    numpy float64 brute force over decoded weights
 *   routing                 reference invariants; numpy stable-sort model
 *   hash routing            closed form
 *   RMSNorm                 closed form; RMS of output is 1
 *   gtmoe_oracle_exp/log1p  restate Go's portable math.Exp / math.Log1p (the
 *                           fdlibm methods); pinned to <= 1 ulp of glibc.  Their
 *                           last-ulp agreement with Go's amd64 Exp assembly is
 *                           parity unpinned (no Go toolchain here).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { PREC_FLOAT64 = 0, PREC_FLOAT32 = 1, PREC_INT8 = 2, PREC_FP4 = 3 };
enum { ACT_LINEAR = 0, ACT_SILU = 1, ACT_CLAMPED_SILU = 2, ACT_CLAMPED_LINEAR = 3 };

#define VALUES_PER_SCALE 16 /* lowprecision/lowprecision.go:46 */

static int scale_blocks(int width) { return (width + VALUES_PER_SCALE - 1) / VALUES_PER_SCALE; }
static int fp4_row_bytes(int width) { return (width + 1) / 2; } /* rows.go:34-36 */

static double from_bits(uint64_t u) { double d; memcpy(&d, &u, sizeof d); return d; }
static uint64_t to_bits(double d) { uint64_t u; memcpy(&u, &d, sizeof u); return u; }

/* ------------------------------------------------------------------------- */
/* Scalar math used on the path.                                              */
/* ------------------------------------------------------------------------- */

/* Go math.Exp, portable form (fdlibm e_exp.c method): x = k ln2 + r with
 * ln2 split into hi/lo, rational approximation of exp(r), then ldexp. */
double gtmoe_oracle_exp(double x)
{
    const double ln2_hi = from_bits(0x3fe62e42fee00000ULL);
    const double ln2_lo = from_bits(0x3dea39ef35793c76ULL);
    const double log2e = from_bits(0x3ff71547652b82feULL);
    const double overflow = 7.09782712893383973096e+02;
    const double underflow = -7.45133219101941108420e+02;
    const double near_zero = 1.0 / (double)(1 << 28);
    const double p1 = from_bits(0x3fc5555555555555ULL);
    const double p2 = from_bits(0xbf66c16c16bebd93ULL);
    const double p3 = from_bits(0x3f11566aaf25de2cULL);
    const double p4 = from_bits(0xbebbbd41c5d26bf1ULL);
    const double p5 = from_bits(0x3e66376972bea4d0ULL);

    if (isnan(x) || (isinf(x) && x > 0)) return x;
    if (isinf(x)) return 0;
    if (x > overflow) return INFINITY;
    if (x < underflow) return 0;
    if (-near_zero < x && x < near_zero) return 1 + x;

    int k = 0;
    if (x < 0) k = (int)(log2e * x - 0.5);
    else if (x > 0) k = (int)(log2e * x + 0.5);
    double hi = x - (double)k * ln2_hi;
    double lo = (double)k * ln2_lo;

    double r = hi - lo;
    double t = r * r;
    double c = r - t * (p1 + t * (p2 + t * (p3 + t * (p4 + t * p5))));
    double y = 1 - ((lo - (r * c) / (2 - c)) - hi);
    return ldexp(y, k);
}

/* Go math.Log1p (fdlibm s_log1p.c method). */
double gtmoe_oracle_log1p(double x)
{
    const double sqrt2m1 = from_bits(0x3fda827999fcef34ULL);
    const double sqrt2halfm1 = from_bits(0xbfd2bec333018866ULL);
    const double small = 1.0 / (double)(1 << 29);
    const double tiny = 1.0 / (double)(1ULL << 54);
    const double two53 = (double)(1ULL << 53);
    const double ln2_hi = from_bits(0x3fe62e42fee00000ULL);
    const double ln2_lo = from_bits(0x3dea39ef35793c76ULL);
    const double lp1 = from_bits(0x3fe5555555555593ULL);
    const double lp2 = from_bits(0x3fd999999997fa04ULL);
    const double lp3 = from_bits(0x3fd2492494229359ULL);
    const double lp4 = from_bits(0x3fcc71c51d8e78afULL);
    const double lp5 = from_bits(0x3fc7466496cb03deULL);
    const double lp6 = from_bits(0x3fc39a09d078c69fULL);
    const double lp7 = from_bits(0x3fc2f112df3e5244ULL);

    if (x < -1 || isnan(x)) return NAN;
    if (x == -1) return -INFINITY;
    if (isinf(x)) return INFINITY;

    double absx = fabs(x);
    double f = 0;
    uint64_t iu = 0;
    int k = 1;
    if (absx < sqrt2m1) {
        if (absx < small) {
            if (absx < tiny) return x;
            return x - x * x * 0.5;
        }
        if (x > sqrt2halfm1) {
            k = 0;
            f = x;
            iu = 1;
        }
    }
    double c = 0;
    if (k != 0) {
        double u;
        if (absx < two53) {
            u = 1.0 + x;
            iu = to_bits(u);
            k = (int)((iu >> 52) - 1023);
            if (k > 0) c = 1.0 - (u - x);
            else c = x - (u - 1.0);
            c /= u;
        } else {
            u = x;
            iu = to_bits(u);
            k = (int)((iu >> 52) - 1023);
            c = 0;
        }
        iu &= 0x000fffffffffffffULL;
        if (iu < 0x0006a09e667f3bcdULL) {
            u = from_bits(iu | 0x3ff0000000000000ULL);
        } else {
            k++;
            u = from_bits(iu | 0x3fe0000000000000ULL);
            iu = (0x0010000000000000ULL - iu) >> 2;
        }
        f = u - 1.0;
    }
    double hfsq = 0.5 * f * f;
    double s, r, z;
    if (iu == 0) {
        if (f == 0) {
            if (k == 0) return 0;
            c += (double)k * ln2_lo;
            return (double)k * ln2_hi + c;
        }
        r = hfsq * (1.0 - 0.66666666666666666 * f);
        if (k == 0) return f - r;
        return (double)k * ln2_hi - ((r - ((double)k * ln2_lo + c)) - f);
    }
    s = f / (2.0 + f);
    z = s * s;
    r = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + r));
    return (double)k * ln2_hi - ((hfsq - (s * (hfsq + r) + ((double)k * ln2_lo + c))) - f);
}

/* activationfunction/moreactivationfunctions.go:8-16 */
double gtmoe_oracle_softplus(double x)
{
    if (x > 20) return x;
    if (x < -20) return gtmoe_oracle_exp(x);
    return gtmoe_oracle_log1p(gtmoe_oracle_exp(x));
}

/* activationfunction/activationfunction.go:35-37, 102-105 */
static double sigmoid(double x) { return 1 / (1 + gtmoe_oracle_exp(-x)); }
double gtmoe_oracle_silu(double x)
{
    double s = sigmoid(x);
    return x * s;
}

/* mixtureofexperts/mixtureofexperts.go:80-82 */
double gtmoe_oracle_affinity(double logit) { return sqrt(gtmoe_oracle_softplus(logit)); }

/* activation dispatch: activationfunction.go:158-170 (Linear), :111-115 (SiLU),
 * moreactivationfunctions.go:207-244 (ClampedSiLU, ClampedLinear) */
static double activate(int activation, double limit, double x)
{
    switch (activation) {
    case ACT_SILU: return gtmoe_oracle_silu(x);
    case ACT_CLAMPED_SILU: return x > limit ? gtmoe_oracle_silu(limit) : gtmoe_oracle_silu(x);
    case ACT_CLAMPED_LINEAR:
        if (x > limit) return limit;
        if (x < -limit) return -limit;
        return x;
    default: return x;
    }
}

/* ------------------------------------------------------------------------- */
/* lowprecision: encode (Rows.Append), decode (Rows.Row), DotRow              */
/* ------------------------------------------------------------------------- */

/* lowprecision.go:66-78 */
static int8_t encode_int8(double value, double scale)
{
    if (scale == 0) return 0;
    double rounded = round(value / scale); /* Go math.Round: half away from zero */
    if (rounded > 127) rounded = 127;
    if (rounded < -127) rounded = -127;
    return (int8_t)rounded;
}

/* lowprecision.go:80-96 */
static uint8_t encode_fp4(double value, double scale)
{
    static const double halfway[7] = {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5};
    if (scale == 0) return 0;
    uint8_t sign = value < 0 ? 8 : 0;
    double scaled = fabs(value) / scale;
    int closest = 0;
    while (closest < 7 && scaled > halfway[closest]) closest++;
    return (uint8_t)(sign | closest);
}

static double block_absmax(const double *values, int n)
{
    double largest = 0.0;
    for (int i = 0; i < n; i++)
        if (fabs(values[i]) > largest) largest = fabs(values[i]);
    return largest;
}

/* Rows.Append over `rows` rows (rows.go:38-79).  Output buffers follow the
 * reference storage: f32[rows*width], i8[rows*width],
 * fp4[rows*ceil(width/2)] (even value in the low nibble), scales[rows*blocks]. */
void gtmoe_oracle_encode_rows(int precision, int rows, int width, const double *values,
                              float *f32_out, int8_t *i8_out, uint8_t *fp4_out, float *scales_out)
{
    int blocks = scale_blocks(width);
    for (int r = 0; r < rows; r++) {
        const double *row = values + (size_t)r * width;
        if (precision == PREC_FLOAT32) {
            for (int i = 0; i < width; i++) f32_out[(size_t)r * width + i] = (float)row[i];
        } else if (precision == PREC_INT8) {
            for (int b = 0; b < blocks; b++) {
                int start = b * VALUES_PER_SCALE;
                int end = start + VALUES_PER_SCALE < width ? start + VALUES_PER_SCALE : width;
                double scale = block_absmax(row + start, end - start) / 127;
                float scale32 = (float)scale;
                scales_out[(size_t)r * blocks + b] = scale32;
                for (int i = start; i < end; i++)
                    i8_out[(size_t)r * width + i] = encode_int8(row[i], (double)scale32);
            }
        } else if (precision == PREC_FP4) {
            int row_bytes = fp4_row_bytes(width);
            uint8_t *packed = fp4_out + (size_t)r * row_bytes;
            memset(packed, 0, (size_t)row_bytes);
            for (int b = 0; b < blocks; b++) {
                int start = b * VALUES_PER_SCALE;
                int end = start + VALUES_PER_SCALE < width ? start + VALUES_PER_SCALE : width;
                double scale = block_absmax(row + start, end - start) / 6;
                float scale32 = (float)scale;
                scales_out[(size_t)r * blocks + b] = scale32;
                for (int i = start; i < end; i++) {
                    uint8_t code = encode_fp4(row[i], (double)scale32);
                    if (i % 2 == 0) packed[i / 2] = code;
                    else packed[i / 2] |= (uint8_t)(code << 4);
                }
            }
        }
    }
}

/* A weight matrix in the reference's Rows storage. */
typedef struct {
    int32_t precision;
    int32_t rows;
    int32_t width;
    int32_t pad_;
    const void *values; /* f64 / f32 / i8 / packed fp4 */
    const float *scales;
} gtmoe_oracle_rows;

static const double fp4_signed[16] = {0, 0.5, 1, 1.5, 2, 3, 4, 6, 0, -0.5, -1, -1.5, -2, -3, -4, -6};
static const double fp4_magnitude[8] = {0, 0.5, 1, 1.5, 2, 3, 4, 6};

static uint8_t fp4_code(const uint8_t *packed_row, int i)
{
    uint8_t packed = packed_row[i / 2];
    return (i % 2 == 1) ? (uint8_t)(packed >> 4) : (uint8_t)(packed & 15);
}

/* Rows.Row (rows.go:87-119) */
void gtmoe_oracle_decode_row(const gtmoe_oracle_rows *m, int index, double *out)
{
    int w = m->width, blocks = scale_blocks(w);
    switch (m->precision) {
    case PREC_FLOAT64:
        memcpy(out, (const double *)m->values + (size_t)index * w, sizeof(double) * (size_t)w);
        break;
    case PREC_FLOAT32:
        for (int i = 0; i < w; i++) out[i] = (double)((const float *)m->values)[(size_t)index * w + i];
        break;
    case PREC_INT8:
        for (int i = 0; i < w; i++) {
            double scale = (double)m->scales[(size_t)index * blocks + i / VALUES_PER_SCALE];
            out[i] = (double)((const int8_t *)m->values)[(size_t)index * w + i] * scale;
        }
        break;
    case PREC_FP4: {
        const uint8_t *row = (const uint8_t *)m->values + (size_t)index * fp4_row_bytes(w);
        for (int i = 0; i < w; i++) {
            uint8_t code = fp4_code(row, i);
            double scale = (double)m->scales[(size_t)index * blocks + i / VALUES_PER_SCALE];
            double value = fp4_magnitude[code & 7] * scale; /* decodeFP4, lowprecision.go:98-104 */
            out[i] = (code & 8) ? -value : value;
        }
        break;
    }
    }
}

/* Rows.DotRow (rows.go:207-257): sequential sums, per-16-block partial sums
 * scaled once per block. */
double gtmoe_oracle_dot_row(const gtmoe_oracle_rows *m, int row, const double *vector)
{
    int w = m->width, blocks = scale_blocks(w);
    double sum = 0.0;
    switch (m->precision) {
    case PREC_FLOAT64: {
        const double *v = (const double *)m->values + (size_t)row * w;
        for (int i = 0; i < w; i++) sum += vector[i] * v[i];
        break;
    }
    case PREC_FLOAT32: {
        const float *v = (const float *)m->values + (size_t)row * w;
        for (int i = 0; i < w; i++) sum += vector[i] * (double)v[i];
        break;
    }
    case PREC_INT8: {
        const int8_t *v = (const int8_t *)m->values + (size_t)row * w;
        for (int b = 0; b < blocks; b++) {
            int start = b * VALUES_PER_SCALE;
            int end = start + VALUES_PER_SCALE < w ? start + VALUES_PER_SCALE : w;
            double block_sum = 0.0;
            for (int i = start; i < end; i++) block_sum += vector[i] * (double)v[i];
            sum += block_sum * (double)m->scales[(size_t)row * blocks + b];
        }
        break;
    }
    case PREC_FP4: {
        const uint8_t *packed = (const uint8_t *)m->values + (size_t)row * fp4_row_bytes(w);
        for (int b = 0; b < blocks; b++) {
            int start = b * VALUES_PER_SCALE;
            int end = start + VALUES_PER_SCALE < w ? start + VALUES_PER_SCALE : w;
            double block_sum = 0.0;
            for (int i = start; i < end; i++) block_sum += vector[i] * fp4_signed[fp4_code(packed, i)];
            sum += block_sum * (double)m->scales[(size_t)row * blocks + b];
        }
        break;
    }
    }
    return sum;
}

/* ------------------------------------------------------------------------- */
/* perceptron.Layer.Forward with the SplitAcrossThreads policy                */
/* ------------------------------------------------------------------------- */

typedef struct {
    gtmoe_oracle_rows weights; /* outputs x inputs */
    const double *biases;      /* outputs */
    int32_t activation;
    int32_t pad_;
    double clamp_limit;
} gtmoe_oracle_layer;

typedef struct {
    const gtmoe_oracle_layer *layer;
    const double *inputs;
    int tokens;
    double *pre; /* tokens x outputs */
    int first, last;
} split_job;

static void *run_split_job(void *arg)
{
    split_job *job = (split_job *)arg;
    int n_out = job->layer->weights.rows, width = job->layer->weights.width;
    /* layer.go:121-131: neuron-major, each (neuron, example) one DotRow */
    for (int neuron = job->first; neuron < job->last; neuron++)
        for (int t = 0; t < job->tokens; t++)
            job->pre[(size_t)t * n_out + neuron] =
                gtmoe_oracle_dot_row(&job->layer->weights, neuron, job->inputs + (size_t)t * width);
    return NULL;
}

/* vectormath/backend.go:56-78 */
#define WORK_BEFORE_MORE_THREADS (64 * 64 * 64)

static void split_across_threads(int threads, int items, long work_per_item, split_job *proto)
{
    if ((long)items * work_per_item < WORK_BEFORE_MORE_THREADS || threads <= 1 || items < 2) {
        proto->first = 0;
        proto->last = items;
        run_split_job(proto);
        return;
    }
    if (threads > items) threads = items;
    int per = (items + threads - 1) / threads;
    int count = (items + per - 1) / per;
    pthread_t *ids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)count);
    split_job *jobs = (split_job *)malloc(sizeof(split_job) * (size_t)count);
    int started = 0;
    for (int c = 0; c < count; c++) {
        jobs[c] = *proto;
        jobs[c].first = c * per;
        jobs[c].last = (c + 1) * per < items ? (c + 1) * per : items;
        if (pthread_create(&ids[c], NULL, run_split_job, &jobs[c]) != 0) {
            run_split_job(&jobs[c]); /* run inline if a thread cannot start */
            ids[c] = 0;
        } else {
            started++;
        }
    }
    for (int c = 0; c < count; c++)
        if (ids[c]) pthread_join(ids[c], NULL);
    (void)started;
    free(ids);
    free(jobs);
}

/* Layer.Forward (layer.go:133-162): pre = x.W^T (DotRow), pre += bias,
 * out = act(pre).  `out` is tokens x outputs. */
void gtmoe_oracle_layer_forward(const gtmoe_oracle_layer *layer, int tokens, const double *inputs,
                                int threads, double *out)
{
    int n_out = layer->weights.rows, width = layer->weights.width;
    double *pre = (double *)malloc(sizeof(double) * (size_t)tokens * n_out + 8);
    split_job job = {layer, inputs, tokens, pre, 0, n_out};
    split_across_threads(threads, n_out, (long)tokens * width, &job);
    for (int t = 0; t < tokens; t++)
        for (int n = 0; n < n_out; n++) {
            double p = pre[(size_t)t * n_out + n] + layer->biases[n];
            out[(size_t)t * n_out + n] = activate(layer->activation, layer->clamp_limit, p);
        }
    free(pre);
}

typedef struct {
    gtmoe_oracle_layer gate, up, down;
} gtmoe_oracle_expert;

/* GatedFeedForward.Forward (feedforward/gatedfeedforward.go:49-57) */
void gtmoe_oracle_expert_forward(const gtmoe_oracle_expert *e, int tokens, const double *inputs,
                                 int threads, double *out)
{
    int hidden = e->gate.weights.rows;
    size_t n = (size_t)tokens * hidden;
    double *g = (double *)malloc(sizeof(double) * n + 8);
    double *u = (double *)malloc(sizeof(double) * n + 8);
    gtmoe_oracle_layer_forward(&e->gate, tokens, inputs, threads, g);
    gtmoe_oracle_layer_forward(&e->up, tokens, inputs, threads, u);
    for (size_t i = 0; i < n; i++) g[i] = g[i] * u[i]; /* MultiplyMatricesEach */
    gtmoe_oracle_layer_forward(&e->down, tokens, g, threads, out);
    free(g);
    free(u);
}

/* ------------------------------------------------------------------------- */
/* Routing                                                                     */
/* ------------------------------------------------------------------------- */

/* sort.SliceStable(candidates, less) of mixtureofexperts.go:106, with
 * less(i, j) = score(candidates[i]) > score(candidates[j]).  Go's stable sort
 * (package sort, stable_func and its helpers insertionSort_func,
 * symMerge_func, rotate_func, swapRange_func; Go 1.27 as go.mod pins it)
 * insertion-sorts blocks of 20 and then merges neighbouring blocks of 20,
 * 40, 80, ... with SymMerge (Kim & Kutzner, 2004).  For scores that are
 * totally ordered every stable sort gives the same order; with NaN scores
 * (no NaN compares greater, or less, than anything) the order is whatever
 * this sequence of comparisons and swaps leaves, so it is followed step for
 * step.  Candidate positions are swapped, as the reference's Swapper does. */
typedef struct {
    int *c;
    const double *s;
} cand_sort;

static int cs_less(const cand_sort *d, int i, int j) { return d->s[d->c[i]] > d->s[d->c[j]]; }

static void cs_swap(const cand_sort *d, int i, int j)
{
    int t = d->c[i];
    d->c[i] = d->c[j];
    d->c[j] = t;
}

static void cs_insertion(const cand_sort *d, int a, int b)
{
    for (int i = a + 1; i < b; i++)
        for (int j = i; j > a && cs_less(d, j, j - 1); j--) cs_swap(d, j, j - 1);
}

static void cs_swap_range(const cand_sort *d, int a, int b, int n)
{
    for (int i = 0; i < n; i++) cs_swap(d, a + i, b + i);
}

/* the blocks [a, m) and [m, b) exchanged */
static void cs_rotate(const cand_sort *d, int a, int m, int b)
{
    int i = m - a, j = b - m;
    while (i != j) {
        if (i > j) {
            cs_swap_range(d, m - i, m, j);
            i -= j;
        } else {
            cs_swap_range(d, m - i, m + j - i, i);
            j -= i;
        }
    }
    cs_swap_range(d, m - i, m, i);
}

/* merges the sorted runs [a, m) and [m, b) */
static void cs_sym_merge(const cand_sort *d, int a, int m, int b)
{
    if (m - a == 1) { /* one element in front: binary search, then move it */
        int i = m, j = b;
        while (i < j) {
            int h = (int)((unsigned)(i + j) >> 1);
            if (cs_less(d, h, a)) i = h + 1;
            else j = h;
        }
        for (int k = a; k < i - 1; k++) cs_swap(d, k, k + 1);
        return;
    }
    if (b - m == 1) { /* one element behind */
        int i = a, j = m;
        while (i < j) {
            int h = (int)((unsigned)(i + j) >> 1);
            if (!cs_less(d, m, h)) i = h + 1;
            else j = h;
        }
        for (int k = m; k > i; k--) cs_swap(d, k, k - 1);
        return;
    }
    int mid = (int)((unsigned)(a + b) >> 1);
    int n = mid + m, start, r;
    if (m > mid) {
        start = n - b;
        r = mid;
    } else {
        start = a;
        r = m;
    }
    int p = n - 1;
    while (start < r) {
        int c = (int)((unsigned)(start + r) >> 1);
        if (!cs_less(d, p - c, c)) start = c + 1;
        else r = c;
    }
    int end = n - start;
    if (start < m && m < end) cs_rotate(d, start, m, end);
    if (a < start && start < mid) cs_sym_merge(d, a, start, mid);
    if (mid < end && end < b) cs_sym_merge(d, mid, end, b);
}

static void cs_stable(const cand_sort *d, int n)
{
    int block = 20, a = 0, b = block;
    while (b <= n) {
        cs_insertion(d, a, b);
        a = b;
        b += block;
    }
    cs_insertion(d, a, n);
    while (block < n) {
        a = 0;
        b = 2 * block;
        while (b <= n) {
            cs_sym_merge(d, a, a + block, b);
            a = b;
            b += 2 * block;
        }
        if (a + block < n) cs_sym_merge(d, a, a + block, n);
        block *= 2;
    }
}

/* The candidate order sort.SliceStable leaves for scores s[0..n) (exported
 * for the tests). */
void gtmoe_oracle_go_stable_order(int n, const double *s, int *order)
{
    for (int e = 0; e < n; e++) order[e] = e;
    cand_sort d = {order, s};
    cs_stable(&d, n);
}

/* routedExperts (mixtureofexperts.go:98-112): stable sort by score descending
 * (ties keep the lower expert index first), take k, sort ascending. */
static void routed_experts(int experts, int k, const double *affinities, const double *balance,
                           int32_t *chosen, int *scratch)
{
    double *score = (double *)malloc(sizeof(double) * (size_t)experts);
    for (int e = 0; e < experts; e++) score[e] = affinities[e] + balance[e]; /* choiceScore */
    gtmoe_oracle_go_stable_order(experts, score, scratch);
    free(score);
    /* sort.Ints on the first k */
    for (int i = 0; i < k; i++) chosen[i] = scratch[i];
    for (int i = 1; i < k; i++) {
        int32_t v = chosen[i];
        int j = i - 1;
        while (j >= 0 && chosen[j] > v) {
            chosen[j + 1] = chosen[j];
            j--;
        }
        chosen[j + 1] = v;
    }
}

/* Learned routing from router logits (mixtureofexperts.go:153-173):
 * affinity = sqrt(softplus(logit)), top-k by affinity + balance bias,
 * gates = affinity / sum of chosen affinities (summed in ascending order). */
void gtmoe_oracle_route_from_logits(int tokens, int experts, int k, const double *logits,
                                    const double *balance, int32_t *chosen, double *gates,
                                    double *affinities)
{
    int *scratch = (int *)malloc(sizeof(int) * (size_t)experts);
    double *aff_local = affinities ? NULL : (double *)malloc(sizeof(double) * (size_t)experts);
    for (int t = 0; t < tokens; t++) {
        double *a = affinities ? affinities + (size_t)t * experts : aff_local;
        for (int e = 0; e < experts; e++) a[e] = gtmoe_oracle_affinity(logits[(size_t)t * experts + e]);
        int32_t *c = chosen + (size_t)t * k;
        routed_experts(experts, k, a, balance, c, scratch);
        double total = 0.0;
        for (int i = 0; i < k; i++) total += a[c[i]];
        for (int i = 0; i < k; i++) gates[(size_t)t * k + i] = a[c[i]] / total;
    }
    free(scratch);
    free(aff_local);
}

/* hashedExperts (mixtureofexperts.go:88-96) and the 1/k gates (:142-152).
 * Returns -1 (the reference panics) if an id is negative. */
int gtmoe_oracle_hash_route(int tokens, int experts, int k, const int64_t *token_ids,
                            int32_t *chosen, double *gates)
{
    for (int t = 0; t < tokens; t++) {
        if (token_ids[t] < 0) return -1;
        uint64_t first = ((uint64_t)token_ids[t] * 2654435761ULL + 12345ULL) % (uint64_t)experts;
        for (int i = 0; i < k; i++) {
            chosen[(size_t)t * k + i] = (int32_t)((first + (uint64_t)i) % (uint64_t)experts);
            gates[(size_t)t * k + i] = 1 / (double)k;
        }
    }
    return 0;
}

/* rowsForExpert / expertLoad (mixtureofexperts.go:175-180, 188-190):
 * offsets[E+1], rows[T*k] = token indices, experts ascending, tokens
 * ascending inside an expert. */
void gtmoe_oracle_dispatch(int tokens, int experts, int k, const int32_t *chosen, int32_t *load,
                           int32_t *offsets, int32_t *rows)
{
    memset(load, 0, sizeof(int32_t) * (size_t)experts);
    for (int t = 0; t < tokens; t++)
        for (int i = 0; i < k; i++) load[chosen[(size_t)t * k + i]]++;
    offsets[0] = 0;
    for (int e = 0; e < experts; e++) offsets[e + 1] = offsets[e] + load[e];
    int32_t *fill = (int32_t *)malloc(sizeof(int32_t) * (size_t)experts + 4);
    for (int e = 0; e < experts; e++) fill[e] = offsets[e];
    for (int t = 0; t < tokens; t++)
        for (int i = 0; i < k; i++) rows[fill[chosen[(size_t)t * k + i]]++] = t;
    free(fill);
}

/* ------------------------------------------------------------------------- */
/* MixtureOfExperts.Forward                                                    */
/* ------------------------------------------------------------------------- */

typedef struct {
    int32_t vector_size;
    int32_t hidden_size;
    int32_t shared_experts;
    int32_t routed_experts;
    int32_t experts_per_token;
    int32_t use_hash_routing;
    const gtmoe_oracle_expert *shared;
    const gtmoe_oracle_expert *routed;
    gtmoe_oracle_layer router;
    const double *balance_biases;
} gtmoe_oracle_moe;

/* Expert outputs and the weighted combine (mixtureofexperts.go:175-205),
 * given chosen experts and gates.  Experts run on gathered rows exactly as
 * the reference does; outputs is tokens x vector_size. */
static void moe_experts_and_combine(const gtmoe_oracle_moe *moe, int tokens, const double *inputs,
                                    const int32_t *chosen, const double *gates, int threads,
                                    double *outputs, int32_t *load_out)
{
    int d = moe->vector_size, E = moe->routed_experts, k = moe->experts_per_token;
    size_t td = (size_t)tokens * d;
    int32_t *load = (int32_t *)malloc(sizeof(int32_t) * (size_t)E + 4);
    int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t *rows = (int32_t *)malloc(sizeof(int32_t) * (size_t)tokens * k + 4);
    gtmoe_oracle_dispatch(tokens, E, k, chosen, load, offsets, rows);
    if (load_out) memcpy(load_out, load, sizeof(int32_t) * (size_t)E);

    /* outputs = 0; outputs = outputs + shared(inputs) for each shared expert */
    for (size_t i = 0; i < td; i++) outputs[i] = 0.0;
    double *tmp = (double *)malloc(sizeof(double) * td + 8);
    for (int s = 0; s < moe->shared_experts; s++) {
        gtmoe_oracle_expert_forward(&moe->shared[s], tokens, inputs, threads, tmp);
        for (size_t i = 0; i < td; i++) outputs[i] = outputs[i] + tmp[i];
    }
    free(tmp);

    /* routed experts over gathered rows */
    double *expert_out = (double *)malloc(sizeof(double) * (size_t)tokens * k * d + 8);
    double *gathered = (double *)malloc(sizeof(double) * (size_t)tokens * d + 8);
    for (int e = 0; e < E; e++) {
        int n = load[e];
        if (n == 0) continue;
        for (int r = 0; r < n; r++)
            memcpy(gathered + (size_t)r * d, inputs + (size_t)rows[offsets[e] + r] * d, sizeof(double) * (size_t)d);
        gtmoe_oracle_expert_forward(&moe->routed[e], n, gathered, threads,
                                    expert_out + (size_t)offsets[e] * d);
    }
    free(gathered);

    /* combine: slots in chosen order; indexOf = position of the token in
     * the expert's ascending token list */
    for (int t = 0; t < tokens; t++) {
        double *out_row = outputs + (size_t)t * d;
        for (int i = 0; i < k; i++) {
            int e = chosen[(size_t)t * k + i];
            int lo = offsets[e], hi = offsets[e + 1] - 1, pos = -1;
            while (lo <= hi) { /* tokens are ascending: binary search == indexOf */
                int mid = (lo + hi) / 2;
                if (rows[mid] == t) { pos = mid; break; }
                if (rows[mid] < t) lo = mid + 1;
                else hi = mid - 1;
            }
            const double *y = expert_out + (size_t)pos * d;
            double g = gates[(size_t)t * k + i];
            for (int j = 0; j < d; j++) out_row[j] += g * y[j];
        }
    }
    free(expert_out);
    free(load);
    free(offsets);
    free(rows);
}

/* Full forward.  Optional outputs (may be NULL): logits/affinities T x E
 * (learned routing only), chosen/gates T x k, load E.  Returns 0, or -1 when
 * the reference would panic (hash routing with a negative id). */
int gtmoe_oracle_moe_forward(const gtmoe_oracle_moe *moe, int tokens, const double *inputs,
                             const int64_t *token_ids, int threads, double *outputs,
                             int32_t *chosen_out, double *gates_out, int32_t *load_out,
                             double *logits_out, double *affinities_out)
{
    int E = moe->routed_experts, k = moe->experts_per_token;
    int32_t *chosen = (int32_t *)malloc(sizeof(int32_t) * (size_t)tokens * k + 4);
    double *gates = (double *)malloc(sizeof(double) * (size_t)tokens * k + 8);
    if (moe->use_hash_routing) {
        if (gtmoe_oracle_hash_route(tokens, E, k, token_ids, chosen, gates) != 0) {
            free(chosen);
            free(gates);
            return -1;
        }
    } else {
        double *logits = (double *)malloc(sizeof(double) * (size_t)tokens * E + 8);
        gtmoe_oracle_layer_forward(&moe->router, tokens, inputs, threads, logits);
        if (logits_out) memcpy(logits_out, logits, sizeof(double) * (size_t)tokens * E);
        gtmoe_oracle_route_from_logits(tokens, E, k, logits, moe->balance_biases, chosen, gates,
                                       affinities_out);
        free(logits);
    }
    moe_experts_and_combine(moe, tokens, inputs, chosen, gates, threads, outputs, load_out);
    if (chosen_out) memcpy(chosen_out, chosen, sizeof(int32_t) * (size_t)tokens * k);
    if (gates_out) memcpy(gates_out, gates, sizeof(double) * (size_t)tokens * k);
    free(chosen);
    free(gates);
    return 0;
}

/* Forward with routing supplied by the caller (chosen/gates T x k): the
 * expert and combine part of the reference under a given routing. */
void gtmoe_oracle_moe_forward_routed(const gtmoe_oracle_moe *moe, int tokens, const double *inputs,
                                     const int32_t *chosen, const double *gates, int threads,
                                     double *outputs, int32_t *load_out)
{
    moe_experts_and_combine(moe, tokens, inputs, chosen, gates, threads, outputs, load_out);
}

/* RMSNorm.Forward (normalization/rmsnorm.go:33-53) */
void gtmoe_oracle_rmsnorm(int tokens, int width, const double *inputs, const double *weights,
                          double epsilon, double *out)
{
    for (int t = 0; t < tokens; t++) {
        const double *x = inputs + (size_t)t * width;
        double dot = 0.0;
        for (int i = 0; i < width; i++) dot += x[i] * x[i];
        double mean = dot / (double)width;
        double rms = sqrt(mean + epsilon);
        for (int i = 0; i < width; i++) out[(size_t)t * width + i] = x[i] / rms * weights[i];
    }
}

/* A stack of blocks without attention (transformer/block.go:71-77):
 * x <- x + MoE(RMSNorm(x)) per layer.  x is updated in place.  The
 * per-layer chosen experts go to chosen_out[layer][T][k] when given. */
int gtmoe_oracle_stack_forward(const gtmoe_oracle_moe *layers, const double *const *norm_weights,
                               int n_layers, int tokens, double *x, const int64_t *token_ids,
                               int threads, int32_t *chosen_out)
{
    for (int l = 0; l < n_layers; l++) {
        const gtmoe_oracle_moe *moe = &layers[l];
        size_t td = (size_t)tokens * moe->vector_size;
        double *normed = (double *)malloc(sizeof(double) * td + 8);
        double *fed = (double *)malloc(sizeof(double) * td + 8);
        gtmoe_oracle_rmsnorm(tokens, moe->vector_size, x, norm_weights[l], 1e-6, normed);
        int32_t *chosen = chosen_out ? chosen_out + (size_t)l * tokens * moe->experts_per_token : NULL;
        int rc = gtmoe_oracle_moe_forward(moe, tokens, normed, token_ids, threads, fed, chosen, NULL,
                                          NULL, NULL, NULL);
        if (rc == 0)
            for (size_t i = 0; i < td; i++) x[i] = x[i] + fed[i];
        free(normed);
        free(fed);
        if (rc != 0) return rc;
    }
    return 0;
}

/* The same stack under routing supplied per layer: chosen/gates are
 * [n_layers][T][k].  Used to compare a device stack layer by layer under the
 * device's own routing. */
void gtmoe_oracle_stack_forward_routed(const gtmoe_oracle_moe *layers, const double *const *norm_weights,
                                       int n_layers, int tokens, double *x, const int32_t *chosen,
                                       const double *gates, int threads)
{
    for (int l = 0; l < n_layers; l++) {
        const gtmoe_oracle_moe *moe = &layers[l];
        size_t td = (size_t)tokens * moe->vector_size;
        size_t tk = (size_t)tokens * moe->experts_per_token;
        double *normed = (double *)malloc(sizeof(double) * td + 8);
        double *fed = (double *)malloc(sizeof(double) * td + 8);
        gtmoe_oracle_rmsnorm(tokens, moe->vector_size, x, norm_weights[l], 1e-6, normed);
        moe_experts_and_combine(moe, tokens, normed, chosen + (size_t)l * tk, gates + (size_t)l * tk,
                                threads, fed, NULL);
        for (size_t i = 0; i < td; i++) x[i] = x[i] + fed[i];
        free(normed);
        free(fed);
    }
}

/* Element-wise evaluation of the scalar functions above over an array, for
 * pinning them against independent implementations.  fn: 0 exp, 1 log1p,
 * 2 softplus, 3 affinity, 4 silu. */
void gtmoe_oracle_map(int fn, long n, const double *in, double *out)
{
    for (long i = 0; i < n; i++) {
        double x = in[i];
        switch (fn) {
        case 0: out[i] = gtmoe_oracle_exp(x); break;
        case 1: out[i] = gtmoe_oracle_log1p(x); break;
        case 2: out[i] = gtmoe_oracle_softplus(x); break;
        case 3: out[i] = gtmoe_oracle_affinity(x); break;
        default: out[i] = gtmoe_oracle_silu(x); break;
        }
    }
}
