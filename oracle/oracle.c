/*
 * CPU oracle for the KV-cached Whisper decoder — TEST INFRASTRUCTURE ONLY.
 * See oracle.h for what each function restates and what pins it. Nothing in
 * the product path loads this file; it is the checker.
 *
 * Build: oracle/Makefile (gcc, no fast-math: the double arithmetic has to keep
 * the reference's operation order).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

int oracle_set_threads(int threads)
{
#ifdef _OPENMP
    if (threads < 1)
        threads = 1;
    g_threads = threads;
    omp_set_num_threads(threads);
#else
    (void) threads;
    g_threads = 1;
#endif
    return g_threads;
}

/* ------------------------------------------------------------------------ */
/* primitives                                                               */
/* ------------------------------------------------------------------------ */

/* Tests/Encoder/Common.h:444-478: mean, then the centred variance, both
 * divided by the width; scale 1/sqrt(var + eps) with the float epsilon
 * widened; (x - mean) * scale * w + b. */
void oracle_layernorm(const double* rows, int row_count, int width,
                      const float* weight, const float* bias, double* out)
{
    for (int row = 0; row < row_count; ++row)
    {
        const double* x = rows + (size_t) row * width;
        double* y = out + (size_t) row * width;
        double mean = 0.0;

        for (int c = 0; c < width; ++c)
            mean += x[c];

        mean /= width;
        double variance = 0.0;

        for (int c = 0; c < width; ++c)
        {
            const double centred = x[c] - mean;
            variance += centred * centred;
        }

        const double scale =
            1.0 / sqrt(variance / width + (double) ORACLE_LAYER_NORM_EPSILON);

        for (int c = 0; c < width; ++c)
            y[c] = (x[c] - mean) * scale * (double) weight[c] + (double) bias[c];
    }
}

/* Tests/Encoder/Common.h:483-505: weight is nn.Linear's [out, inner]; the bias
 * starts the sum and k runs ascending. Parallel over independent outputs. */
void oracle_linear(const double* input, int row_count, int inner,
                   const float* weight, const float* bias_or_null,
                   int output_width, double* out)
{
    const long long total = (long long) row_count * output_width;

#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (g_threads > 1 && total * inner > 65536)
#endif
    for (long long element = 0; element < total; ++element)
    {
        const int row = (int) (element / output_width);
        const int column = (int) (element % output_width);
        const double* x = input + (size_t) row * inner;
        const float* w = weight + (size_t) column * inner;
        double sum = bias_or_null == NULL ? 0.0 : (double) bias_or_null[column];

        for (int k = 0; k < inner; ++k)
            sum += x[k] * (double) w[k];

        out[(size_t) row * output_width + column] = sum;
    }
}

/* Tests/Decoder/Common.h:263-325. scale = 1/sqrt(headWidth) in double, applied
 * to the summed dot product; max over the visible keys; exp(s - max); the
 * weighted value sum divided by the total. */
void oracle_attention(const double* queries, int query_count, int first_query,
                      const double* keys, const double* values, int key_count,
                      int width, int heads, int causal, double* out)
{
    const int head_width = width / heads;
    const double scale = 1.0 / sqrt((double) head_width);
    const long long units = (long long) heads * query_count;

#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (g_threads > 1 && units > 1 && (long long) key_count * width > 4096)
#endif
    for (long long unit = 0; unit < units; ++unit)
    {
        const int head = (int) (unit / query_count);
        const int query = (int) (unit % query_count);
        const int head_column = head * head_width;
        int visible = causal ? first_query + query + 1 : key_count;

        if (visible > key_count)
            visible = key_count;

        double* row = (double*) malloc(sizeof(double) * (size_t) (visible > 0 ? visible : 1));
        double largest = -INFINITY;

        for (int key = 0; key < visible; ++key)
        {
            double total = 0.0;

            for (int c = 0; c < head_width; ++c)
                total += queries[(size_t) query * width + head_column + c]
                         * keys[(size_t) key * width + head_column + c];

            row[key] = scale * total;
            largest = row[key] > largest ? row[key] : largest;
        }

        double total = 0.0;

        for (int key = 0; key < visible; ++key)
        {
            row[key] = exp(row[key] - largest);
            total += row[key];
        }

        for (int c = 0; c < head_width; ++c)
        {
            double weighted = 0.0;

            for (int key = 0; key < visible; ++key)
                weighted += row[key] * values[(size_t) key * width + head_column + c];

            out[(size_t) query * width + head_column + c] = weighted / total;
        }

        free(row);
    }
}

/* Tests/Encoder/Common.h:390-393 */
double oracle_gelu(double x)
{
    return 0.5 * x * (1.0 + erf(x / sqrt(2.0)));
}

/* Tests/Kernels/ArgmaxTests.cpp:12-36 and Tests/Decoder/Common.h:490-500:
 * strict > while scanning forwards, so ties keep the lowest index. */
uint32_t oracle_argmax_masked(const double* row, const float* mask_or_null,
                              int row_length)
{
    int best = -1;

    for (int index = 0; index < row_length; ++index)
    {
        if (mask_or_null != NULL && mask_or_null[index] != 0.f)
            continue;

        if (best < 0 || row[index] > row[best])
            best = index;
    }

    return (uint32_t) (best < 0 ? 0 : best);
}

uint32_t oracle_argmax_masked_f32(const float* row, const float* mask_or_null,
                                  int row_length)
{
    int best = -1;

    for (int index = 0; index < row_length; ++index)
    {
        if (mask_or_null != NULL && mask_or_null[index] != 0.f)
            continue;

        if (best < 0 || row[index] > row[best])
            best = index;
    }

    return (uint32_t) (best < 0 ? 0 : best);
}

/* Kernels/Embed.h:5-15 and Tests/Decoder/Common.h:377-383 (no sqrt(d)). */
void oracle_embed(const uint32_t* tokens, int count, const float* token_table,
                  const float* position_table, int first_position, int width,
                  double* out)
{
    for (int t = 0; t < count; ++t)
        for (int c = 0; c < width; ++c)
            out[(size_t) t * width + c] =
                (double) token_table[(size_t) tokens[t] * width + c]
                + (double) position_table[(size_t) (first_position + t) * width + c];
}

/* ------------------------------------------------------------------------ */
/* storage conversions                                                      */
/* ------------------------------------------------------------------------ */

/* Round to nearest, ties to even, with subnormals, overflow to infinity and
 * NaN kept quiet — the semantics of Core/Utils/Half.cpp:8-55 extended to the
 * whole float range. */
uint16_t oracle_f32_to_f16_bits(float value)
{
    uint32_t x;
    memcpy(&x, &value, sizeof(x));

    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t mag = x & 0x7FFFFFFFu;

    if (mag >= 0x7F800000u)
        return (uint16_t) (mag == 0x7F800000u ? (sign | 0x7C00u)
                                              : (sign | 0x7E00u | ((mag >> 13) & 0x3FFu)));

    if (mag >= 0x477FF000u) /* 65520 and above round to infinity */
        return (uint16_t) (sign | 0x7C00u);

    if (mag < 0x38800000u) /* below 2^-14: an fp16 subnormal or zero */
    {
        if (mag < 0x33000000u) /* below 2^-25: rounds to zero */
            return (uint16_t) sign;

        const uint32_t exponent = mag >> 23;
        const uint32_t significand = (mag & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - exponent;
        uint32_t k = significand >> shift;
        const uint32_t remainder = significand & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);

        if (remainder > half || (remainder == half && (k & 1u)))
            ++k;

        return (uint16_t) (sign | k);
    }

    uint32_t h = (mag >> 13) - (112u << 10);
    const uint32_t remainder = mag & 0x1FFFu;

    if (remainder > 0x1000u || (remainder == 0x1000u && (h & 1u)))
        ++h;

    return (uint16_t) (sign | h);
}

float oracle_f16_bits_to_f32(uint16_t bits)
{
    const uint32_t sign = (uint32_t) (bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    uint32_t x;

    if (exponent == 0x1Fu)
        x = sign | 0x7F800000u | (mantissa << 13);
    else if (exponent != 0)
        x = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    else if (mantissa == 0)
        x = sign;
    else
    {
        /* subnormal: mantissa * 2^-24, normalised */
        int e = -1;

        do
        {
            ++e;
            mantissa <<= 1;
        } while ((mantissa & 0x400u) == 0);

        x = sign | ((uint32_t) (112 - e) << 23) | ((mantissa & 0x3FFu) << 13);
    }

    float value;
    memcpy(&value, &x, sizeof(value));
    return value;
}

uint16_t oracle_f32_to_bf16_bits(float value)
{
    uint32_t x;
    memcpy(&x, &value, sizeof(x));

    if ((x & 0x7FFFFFFFu) > 0x7F800000u)
        return (uint16_t) ((x >> 16) | 0x40u);

    return (uint16_t) ((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

float oracle_bf16_bits_to_f32(uint16_t bits)
{
    const uint32_t x = (uint32_t) bits << 16;
    float value;
    memcpy(&value, &x, sizeof(value));
    return value;
}

/* ------------------------------------------------------------------------ */
/* mt19937 (the standard's 32-bit Mersenne twister)                          */
/* ------------------------------------------------------------------------ */

void oracle_mt19937_fill(uint32_t seed, int64_t count, uint32_t* out)
{
    uint32_t state[624];
    int index = 624;

    state[0] = seed;

    for (int i = 1; i < 624; ++i)
        state[i] = 1812433253u * (state[i - 1] ^ (state[i - 1] >> 30)) + (uint32_t) i;

    for (int64_t n = 0; n < count; ++n)
    {
        if (index >= 624)
        {
            for (int i = 0; i < 624; ++i)
            {
                const uint32_t y = (state[i] & 0x80000000u) | (state[(i + 1) % 624] & 0x7FFFFFFFu);
                state[i] = state[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
            }

            index = 0;
        }

        uint32_t y = state[index++];
        y ^= y >> 11;
        y ^= (y << 7) & 0x9D2C5680u;
        y ^= (y << 15) & 0xEFC60000u;
        y ^= y >> 18;
        out[n] = y;
    }
}

/* ------------------------------------------------------------------------ */
/* the decoder                                                              */
/* ------------------------------------------------------------------------ */

static const float* layer_tensor(const float* const* tensors, int layer, int which)
{
    return tensors[ORACLE_MODEL_TENSORS + layer * ORACLE_TENSORS_PER_LAYER + which];
}

static double* alloc_doubles(size_t count)
{
    return (double*) calloc(count > 0 ? count : 1, sizeof(double));
}

/* One attention sublayer of Tests/Decoder/Common.h:394-437 over `count` rows
 * that stand at absolute positions first..first+count-1:
 *   normalised = LN(hidden); q = Wq·n + bq; k,v appended from n (self) or
 *   taken from the cross cache; hidden += Wo·attention + bo.
 * For self attention the new key and value rows land at cache rows
 * first..first+count-1 before the attention reads rows 0..first+count-1. */
static void attend(const oracle_shape* shape, const float* const* tensors, int layer,
                   int cross, double* hidden, int count, int first,
                   double* key_cache, double* value_cache, int key_count)
{
    const int width = shape->width;
    const int base = cross ? ORACLE_L_CROSS_NORM_W : ORACLE_L_SELF_NORM_W;
    const size_t rows = (size_t) count * width;

    double* normalised = alloc_doubles(rows);
    double* queries = alloc_doubles(rows);
    double* attended = alloc_doubles(rows);
    double* projected = alloc_doubles(rows);

    oracle_layernorm(hidden, count, width, layer_tensor(tensors, layer, base + 0),
                     layer_tensor(tensors, layer, base + 1), normalised);
    oracle_linear(normalised, count, width, layer_tensor(tensors, layer, base + 2),
                  layer_tensor(tensors, layer, base + 3), width, queries);

    if (!cross)
    {
        oracle_linear(normalised, count, width, layer_tensor(tensors, layer, base + 4),
                      NULL, width, key_cache + (size_t) first * width);
        oracle_linear(normalised, count, width, layer_tensor(tensors, layer, base + 5),
                      layer_tensor(tensors, layer, base + 6), width,
                      value_cache + (size_t) first * width);
        key_count = first + count;
    }

    oracle_attention(queries, count, first, key_cache, value_cache, key_count, width,
                     shape->heads, !cross, attended);
    oracle_linear(attended, count, width, layer_tensor(tensors, layer, base + 7),
                  layer_tensor(tensors, layer, base + 8), width, projected);

    for (size_t i = 0; i < rows; ++i)
        hidden[i] += projected[i];

    free(normalised);
    free(queries);
    free(attended);
    free(projected);
}

/* Tests/Decoder/Common.h:439-456: h += fc2(gelu(fc1(LN(h)))). */
static void feed_forward(const oracle_shape* shape, const float* const* tensors,
                         int layer, double* hidden, int count)
{
    const int width = shape->width;
    const int ffn = shape->feed_forward_width;
    double* normalised = alloc_doubles((size_t) count * width);
    double* inner = alloc_doubles((size_t) count * ffn);
    double* projected = alloc_doubles((size_t) count * width);

    oracle_layernorm(hidden, count, width, layer_tensor(tensors, layer, ORACLE_L_FINAL_NORM_W),
                     layer_tensor(tensors, layer, ORACLE_L_FINAL_NORM_B), normalised);
    oracle_linear(normalised, count, width, layer_tensor(tensors, layer, ORACLE_L_FC1_W),
                  layer_tensor(tensors, layer, ORACLE_L_FC1_B), ffn, inner);

    for (size_t i = 0; i < (size_t) count * ffn; ++i)
        inner[i] = oracle_gelu(inner[i]);

    oracle_linear(inner, count, ffn, layer_tensor(tensors, layer, ORACLE_L_FC2_W),
                  layer_tensor(tensors, layer, ORACLE_L_FC2_B), width, projected);

    for (size_t i = 0; i < (size_t) count * width; ++i)
        hidden[i] += projected[i];

    free(normalised);
    free(inner);
    free(projected);
}

struct oracle_session
{
    oracle_shape shape;
    const float* const* tensors;
    int position;
    int cross_rows;
    double** self_keys;
    double** self_values;
    double** cross_keys;
    double** cross_values;
};

oracle_session* oracle_session_create(const oracle_shape* shape,
                                      const float* const* tensors)
{
    oracle_session* s = (oracle_session*) calloc(1, sizeof(oracle_session));
    s->shape = *shape;
    s->tensors = tensors;
    s->self_keys = (double**) calloc((size_t) shape->layers, sizeof(double*));
    s->self_values = (double**) calloc((size_t) shape->layers, sizeof(double*));
    s->cross_keys = (double**) calloc((size_t) shape->layers, sizeof(double*));
    s->cross_values = (double**) calloc((size_t) shape->layers, sizeof(double*));

    for (int l = 0; l < shape->layers; ++l)
    {
        s->self_keys[l] = alloc_doubles((size_t) shape->max_positions * shape->width);
        s->self_values[l] = alloc_doubles((size_t) shape->max_positions * shape->width);
        s->cross_keys[l] = alloc_doubles((size_t) shape->cross_positions * shape->width);
        s->cross_values[l] = alloc_doubles((size_t) shape->cross_positions * shape->width);
    }

    s->cross_rows = shape->cross_positions;
    return s;
}

void oracle_session_destroy(oracle_session* s)
{
    if (s == NULL)
        return;

    for (int l = 0; l < s->shape.layers; ++l)
    {
        free(s->self_keys[l]);
        free(s->self_values[l]);
        free(s->cross_keys[l]);
        free(s->cross_values[l]);
    }

    free(s->self_keys);
    free(s->self_values);
    free(s->cross_keys);
    free(s->cross_values);
    free(s);
}

/* Decoder/Decoder.cpp:121-146, 241-268 with the reference oracle's cross keys
 * and values (Tests/Decoder/Common.h:404-418): projected from the encoder's
 * rows unnormalised, k without bias. */
int oracle_session_begin(oracle_session* s, const float* encoder_rows, int rows)
{
    const int width = s->shape.width;

    if (rows < 0 || rows > s->shape.cross_positions)
        return -1;

    if (rows == 0)
        rows = s->shape.cross_positions;

    double* source = alloc_doubles((size_t) rows * width);

    for (size_t i = 0; i < (size_t) rows * width; ++i)
        source[i] = (double) encoder_rows[i];

    for (int l = 0; l < s->shape.layers; ++l)
    {
        oracle_linear(source, rows, width, layer_tensor(s->tensors, l, ORACLE_L_CROSS_K_W),
                      NULL, width, s->cross_keys[l]);
        oracle_linear(source, rows, width, layer_tensor(s->tensors, l, ORACLE_L_CROSS_V_W),
                      layer_tensor(s->tensors, l, ORACLE_L_CROSS_V_B), width,
                      s->cross_values[l]);
    }

    free(source);
    s->cross_rows = rows;
    s->position = 0;
    return 0;
}

int oracle_session_position(const oracle_session* s)
{
    return s->position;
}

int oracle_session_step(oracle_session* s, const int* tokens, int count,
                        double* hidden_out, double* logits_out)
{
    const oracle_shape* shape = &s->shape;
    const int width = shape->width;

    if (count <= 0 || s->position + count > shape->max_positions)
        return -1;

    double* hidden = alloc_doubles((size_t) count * width);

    for (int t = 0; t < count; ++t)
        for (int c = 0; c < width; ++c)
            hidden[(size_t) t * width + c] =
                (double) s->tensors[ORACLE_EMBED_TOKENS][(size_t) tokens[t] * width + c]
                + (double) s->tensors[ORACLE_EMBED_POSITIONS][(size_t) (s->position + t) * width + c];

    for (int l = 0; l < shape->layers; ++l)
    {
        attend(shape, s->tensors, l, 0, hidden, count, s->position, s->self_keys[l],
               s->self_values[l], 0);
        attend(shape, s->tensors, l, 1, hidden, count, s->position, s->cross_keys[l],
               s->cross_values[l], s->cross_rows);
        feed_forward(shape, s->tensors, l, hidden, count);
    }

    double* final_rows = alloc_doubles((size_t) count * width);
    oracle_layernorm(hidden, count, width, s->tensors[ORACLE_FINAL_NORM_W],
                     s->tensors[ORACLE_FINAL_NORM_B], final_rows);

    if (hidden_out != NULL)
        memcpy(hidden_out, final_rows, sizeof(double) * (size_t) count * width);

    if (logits_out != NULL)
        oracle_linear(final_rows, count, width, s->tensors[ORACLE_EMBED_TOKENS], NULL,
                      shape->vocabulary_size, logits_out);

    free(final_rows);
    free(hidden);
    s->position += count;
    return 0;
}

/* Tests/Decoder/Common.h:360-468: the whole sequence from position 0, the
 * cross keys and values from `encoder_row_count` encoder rows. */
int oracle_decode_full(const oracle_shape* shape, const float* const* tensors,
                       const float* encoder_rows, int encoder_row_count,
                       const int* tokens, int count, double* hidden_out,
                       double* logits_out)
{
    oracle_session* s = oracle_session_create(shape, tensors);
    int status = oracle_session_begin(s, encoder_rows, encoder_row_count);

    if (status == 0)
        status = oracle_session_step(s, tokens, count, hidden_out, logits_out);

    oracle_session_destroy(s);
    return status;
}

int oracle_greedy(oracle_session* s, const int* prompt, int prompt_count, int steps,
                  const float* mask_or_null, int* tokens_out, double* margins_or_null,
                  double* last_logits_or_null)
{
    const int vocab = s->shape.vocabulary_size;
    double* logits = alloc_doubles((size_t) prompt_count * vocab);
    int status = 0;

    for (int step = 0; step < steps; ++step)
    {
        const int rows = step == 0 ? prompt_count : 1;
        const int* feed = step == 0 ? prompt : &tokens_out[step - 1];

        status = oracle_session_step(s, feed, rows, NULL, logits);

        if (status != 0)
            break;

        const double* row = logits + (size_t) (rows - 1) * vocab;
        const uint32_t best = oracle_argmax_masked(row, mask_or_null, vocab);
        tokens_out[step] = (int) best;

        if (margins_or_null != NULL)
        {
            double second = -INFINITY;

            for (int j = 0; j < vocab; ++j)
                if (j != (int) best && (mask_or_null == NULL || mask_or_null[j] == 0.f)
                    && row[j] > second)
                    second = row[j];

            margins_or_null[step] = row[best] - second;
        }

        if (last_logits_or_null != NULL && step == steps - 1)
            memcpy(last_logits_or_null, row, sizeof(double) * (size_t) vocab);
    }

    free(logits);
    return status;
}

/* ------------------------------------------------------------------------ */
/* The encoder                                                               */
/* ------------------------------------------------------------------------ */

int oracle_conv1d_output_length(int input_length, int stride)
{
    return (input_length + 2 * 1 - 3) / stride + 1;
}

/* Tests/Encoder/Common.h:398-441 */
void oracle_conv1d(const double* input, int input_channels, int input_length,
                   const float* weight, const float* bias, int output_channels,
                   int stride, double* out)
{
    const int output_length = oracle_conv1d_output_length(input_length, stride);
    const long long total = (long long) output_channels * output_length;

#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (g_threads > 1 && total * input_channels > 65536)
#endif
    for (long long element = 0; element < total; ++element)
    {
        const int channel = (int) (element / output_length);
        const int frame = (int) (element % output_length);
        double sum = (double) bias[channel];

        for (int source = 0; source < input_channels; ++source)
            for (int tap = 0; tap < 3; ++tap)
            {
                const int at = frame * stride + tap - 1;
                if (at < 0 || at >= input_length)
                    continue;
                sum += (double) weight[((size_t) channel * input_channels + source) * 3 + tap]
                       * input[(size_t) source * input_length + at];
            }
        out[(size_t) channel * output_length + frame] = sum;
    }
}

static const float* encoder_layer_tensor(const float* const* tensors, int layer, int which)
{
    return tensors[ORACLE_ENC_MODEL_TENSORS + layer * ORACLE_ENC_TENSORS_PER_LAYER + which];
}

/* Tests/Encoder/Common.h:596-688 */
int oracle_encode(const oracle_encoder_shape* shape, const float* const* tensors,
                  const float* mel, double* out)
{
    const int width = shape->width, bins = shape->mel_bins, frames = shape->input_frames;
    const int f = shape->feed_forward_width;
    const int conv_frames = oracle_conv1d_output_length(frames, 1);
    const int positions = oracle_conv1d_output_length(conv_frames, 2);
    if (width <= 0 || shape->heads <= 0 || width % shape->heads != 0 || positions <= 0)
        return -1;

    double* input = alloc_doubles((size_t) bins * frames);
    double* convolved = alloc_doubles((size_t) width * conv_frames);
    double* projected = alloc_doubles((size_t) width * positions);
    double* hidden = alloc_doubles((size_t) positions * width);
    double* normalised = alloc_doubles((size_t) positions * width);
    double* queries = alloc_doubles((size_t) positions * width);
    double* keys = alloc_doubles((size_t) positions * width);
    double* values = alloc_doubles((size_t) positions * width);
    double* attended = alloc_doubles((size_t) positions * width);
    double* projection = alloc_doubles((size_t) positions * width);
    double* feed = alloc_doubles((size_t) positions * f);

    for (size_t i = 0; i < (size_t) bins * frames; ++i)
        input[i] = mel[i];

    oracle_conv1d(input, bins, frames, tensors[ORACLE_ENC_CONV1_W], tensors[ORACLE_ENC_CONV1_B], width, 1,
                  convolved);
    for (size_t i = 0; i < (size_t) width * conv_frames; ++i)
        convolved[i] = oracle_gelu(convolved[i]);
    oracle_conv1d(convolved, width, conv_frames, tensors[ORACLE_ENC_CONV2_W], tensors[ORACLE_ENC_CONV2_B], width,
                  2, projected);
    for (size_t i = 0; i < (size_t) width * positions; ++i)
        projected[i] = oracle_gelu(projected[i]);

    /* channel-major out of the convolution, row-major into the transformer */
    const float* table = tensors[ORACLE_ENC_POSITIONS];
    for (int p = 0; p < positions; ++p)
        for (int c = 0; c < width; ++c)
            hidden[(size_t) p * width + c] = projected[(size_t) c * positions + p] + table[(size_t) p * width + c];

    for (int l = 0; l < shape->layers; ++l)
    {
        oracle_layernorm(hidden, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_ATTN_NORM_W),
                         encoder_layer_tensor(tensors, l, ORACLE_EL_ATTN_NORM_B), normalised);
        oracle_linear(normalised, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_Q_W),
                      encoder_layer_tensor(tensors, l, ORACLE_EL_Q_B), width, queries);
        oracle_linear(normalised, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_K_W), NULL, width,
                      keys);
        oracle_linear(normalised, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_V_W),
                      encoder_layer_tensor(tensors, l, ORACLE_EL_V_B), width, values);
        oracle_attention(queries, positions, 0, keys, values, positions, width, shape->heads, 0, attended);
        oracle_linear(attended, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_O_W),
                      encoder_layer_tensor(tensors, l, ORACLE_EL_O_B), width, projection);
        for (size_t i = 0; i < (size_t) positions * width; ++i)
            hidden[i] += projection[i];

        oracle_layernorm(hidden, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_FINAL_NORM_W),
                         encoder_layer_tensor(tensors, l, ORACLE_EL_FINAL_NORM_B), normalised);
        oracle_linear(normalised, positions, width, encoder_layer_tensor(tensors, l, ORACLE_EL_FC1_W),
                      encoder_layer_tensor(tensors, l, ORACLE_EL_FC1_B), f, feed);
        for (size_t i = 0; i < (size_t) positions * f; ++i)
            feed[i] = oracle_gelu(feed[i]);
        oracle_linear(feed, positions, f, encoder_layer_tensor(tensors, l, ORACLE_EL_FC2_W),
                      encoder_layer_tensor(tensors, l, ORACLE_EL_FC2_B), width, projection);
        for (size_t i = 0; i < (size_t) positions * width; ++i)
            hidden[i] += projection[i];
    }

    oracle_layernorm(hidden, positions, width, tensors[ORACLE_ENC_FINAL_NORM_W], tensors[ORACLE_ENC_FINAL_NORM_B],
                     out);

    free(input);
    free(convolved);
    free(projected);
    free(hidden);
    free(normalised);
    free(queries);
    free(keys);
    free(values);
    free(attended);
    free(projection);
    free(feed);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* The mel front end (Tests/Mel/ScalarMel.h:14-134)                          */
/* ------------------------------------------------------------------------ */

int oracle_mel_spectrogram(const float* samples, int sample_count, const float* filters, int fft_length,
                           int hop_length, int frame_count, int mel_count, double* out)
{
    const int pad = fft_length / 2, bins = fft_length / 2 + 1;
    if (sample_count <= pad || fft_length <= 0 || hop_length <= 0 || frame_count <= 0 || mel_count <= 0)
        return -1;
    const double two_pi = 2.0 * 3.14159265358979323846;
    double* window = alloc_doubles((size_t) fft_length);
    double* padded = alloc_doubles((size_t) sample_count + 2 * (size_t) pad);
    double* power = alloc_doubles((size_t) frame_count * bins);

    for (int n = 0; n < fft_length; ++n)
        window[n] = 0.5 * (1.0 - cos(two_pi * n / fft_length));
    /* numpy "reflect": mirrors about the first and last sample, neither repeated */
    for (int i = 0; i < pad; ++i)
        padded[i] = samples[pad - i];
    for (int i = 0; i < sample_count; ++i)
        padded[pad + i] = samples[i];
    for (int i = 0; i < pad; ++i)
        padded[pad + sample_count + i] = samples[sample_count - 2 - i];

#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (g_threads > 1)
#endif
    for (int frame = 0; frame < frame_count; ++frame)
        for (int bin = 0; bin < bins; ++bin)
        {
            double re = 0.0, im = 0.0;
            for (int tap = 0; tap < fft_length; ++tap)
            {
                const double a = padded[(size_t) frame * hop_length + tap] * window[tap];
                const double angle = two_pi * bin * tap / fft_length;
                re += a * cos(angle);
                im -= a * sin(angle);
            }
            power[(size_t) frame * bins + bin] = re * re + im * im;
        }

    double peak = -INFINITY;
    for (int band = 0; band < mel_count; ++band)
        for (int frame = 0; frame < frame_count; ++frame)
        {
            double total = 0.0;
            for (int bin = 0; bin < bins; ++bin)
                total += (double) filters[(size_t) band * bins + bin] * power[(size_t) frame * bins + bin];
            const double v = log10(total > 1e-10 ? total : 1e-10);
            out[(size_t) band * frame_count + frame] = v;
            peak = v > peak ? v : peak;
        }
    for (size_t i = 0; i < (size_t) mel_count * frame_count; ++i)
    {
        const double v = out[i] > peak - 8.0 ? out[i] : peak - 8.0;
        out[i] = (v + 4.0) / 4.0;
    }
    free(window);
    free(padded);
    free(power);
    return 0;
}
