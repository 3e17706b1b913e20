/*
 * CPU oracle for the KV-cached Whisper decoder token loop — TEST INFRASTRUCTURE.
 *
 * This is a restatement, in plain C and double precision, of the reference's
 * scalar decoder oracle (Tests/Decoder/Common.h:202-509 and the helpers it
 * borrows from Tests/Encoder/Common.h:390-505, Tests/Kernels/ArgmaxTests.cpp:
 * 12-36). It is the checker the HIP path is compared against and nothing else:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * The product library never links, loads or falls back to it.
 *
 * Parity pins (each function is checked by something other than itself):
 *   oracle_decode_full     tests/golden fixtures written by an independent
 *                          torch float64 model built from library ops
 *                          (layer_norm, exact gelu, softmax), plus the
 *                          reference's four self-properties (finite, causal
 *                          bit-identical, tied logits to 1e-12, reads the
 *                          encoder: Tests/Decoder/ReferenceDecoderTests.cpp).
 *   oracle_session_*       bitwise equal to oracle_decode_full (same per-row
 *                          operation order), tested for prompts, single steps,
 *                          mixed steps and reduced cross positions.
 *   oracle_layernorm       constant row -> bias (Tests/Kernels/LayerNormTests.cpp
 *                          :101-140); torch.layer_norm in float64.
 *   oracle_attention       one key -> V row; equal scores average V; causal
 *                          weights exact zeros; torch softmax in float64.
 *   oracle_gelu            math.erf closed form; gelu(0)=0, odd-part identity.
 *   oracle_argmax_masked   the reference's hand-built rows and suppression
 *                          cases (Tests/Kernels/ArgmaxTests.cpp:116-233).
 *   oracle_embed           counted tables give exact integers + quarters
 *                          (Tests/Kernels/EmbedTests.cpp:66-205).
 *   oracle_f16/bf16 bits   numpy float16 / torch bfloat16 conversions over
 *                          every finite pattern class.
 *   oracle_mt19937_fill    the C++ standard's known answer (10000th draw of a
 *                          5489-seeded engine is 4123659995).
 *   oracle_conv1d          hand-worked taps (identity kernel, the padded
 *                          ends, stride two) and torch conv1d in float64.
 *   oracle_mel_spectrogram numpy rfft power spectrum, the librosa-style log
 *                          and clamp written independently in the test.
 *   oracle_encode          tests/golden fixture from an independent torch
 *                          float64 encoder (conv1d, gelu, layer_norm,
 *                          softmax), and the reduced-context property
 *                          (Tests/Encoder/EncoderTests.cpp:259-304).
 *
 * Tensors are passed as one array of float pointers in the canonical order
 * below (floats are the stored weights widened exactly, as the reference's
 * readReferenceDecoderModel does at Tests/Decoder/Common.h:214-256).
 */
#ifndef WSP_ORACLE_H
#define WSP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct oracle_shape
{
    int width;
    int heads;
    int layers;
    int feed_forward_width;
    int vocabulary_size;
    int max_positions;
    int cross_positions;
} oracle_shape;

/* Canonical tensor order. Model-level tensors come first, then
 * ORACLE_TENSORS_PER_LAYER per layer. */
enum
{
    ORACLE_EMBED_TOKENS = 0,
    ORACLE_EMBED_POSITIONS = 1,
    ORACLE_FINAL_NORM_W = 2,
    ORACLE_FINAL_NORM_B = 3,
    ORACLE_MODEL_TENSORS = 4
};

enum
{
    /* self attention */
    ORACLE_L_SELF_NORM_W = 0,
    ORACLE_L_SELF_NORM_B,
    ORACLE_L_SELF_Q_W,
    ORACLE_L_SELF_Q_B,
    ORACLE_L_SELF_K_W,
    ORACLE_L_SELF_V_W,
    ORACLE_L_SELF_V_B,
    ORACLE_L_SELF_O_W,
    ORACLE_L_SELF_O_B,
    /* cross attention */
    ORACLE_L_CROSS_NORM_W,
    ORACLE_L_CROSS_NORM_B,
    ORACLE_L_CROSS_Q_W,
    ORACLE_L_CROSS_Q_B,
    ORACLE_L_CROSS_K_W,
    ORACLE_L_CROSS_V_W,
    ORACLE_L_CROSS_V_B,
    ORACLE_L_CROSS_O_W,
    ORACLE_L_CROSS_O_B,
    /* feed forward */
    ORACLE_L_FINAL_NORM_W,
    ORACLE_L_FINAL_NORM_B,
    ORACLE_L_FC1_W,
    ORACLE_L_FC1_B,
    ORACLE_L_FC2_W,
    ORACLE_L_FC2_B,
    ORACLE_TENSORS_PER_LAYER
};

/* The float LayerNorm epsilon the reference widens to double
 * (Kernels/LayerNorm.h:21, Tests/Encoder/Common.h:444-478). */
#define ORACLE_LAYER_NORM_EPSILON 1e-5f

/* Threads used by the parallel loops (1 = the reference's own scalar model).
 * Every parallel loop splits over independent outputs, so results are
 * bit-identical at any thread count. Returns the count in effect. */
int oracle_set_threads(int threads);

/* ---- primitives (each a function of the reference's test helpers) ---- */

/* Tests/Encoder/Common.h:444-478 */
void oracle_layernorm(const double* rows, int row_count, int width,
                      const float* weight, const float* bias, double* out);

/* Tests/Encoder/Common.h:483-505: bias first, then the sum over k ascending. */
void oracle_linear(const double* input, int row_count, int inner,
                   const float* weight, const float* bias_or_null,
                   int output_width, double* out);

/* Tests/Decoder/Common.h:263-325, generalised to a query block that starts at
 * absolute position first_query (query i sees keys 0..first_query+i when
 * causal; the reference's full recompute is first_query = 0). */
void oracle_attention(const double* queries, int query_count, int first_query,
                      const double* keys, const double* values, int key_count,
                      int width, int heads, int causal, double* out);

/* Tests/Encoder/Common.h:390-393 */
double oracle_gelu(double x);

/* Tests/Kernels/ArgmaxTests.cpp:12-36: first index of the largest unmasked
 * value; all masked gives 0. mask may be null (nothing suppressed). */
uint32_t oracle_argmax_masked(const double* row, const float* mask_or_null,
                              int row_length);
uint32_t oracle_argmax_masked_f32(const float* row, const float* mask_or_null,
                                  int row_length);

/* Kernels/Embed.h:5-15: out[t,c] = tok[tokens[t], c] + pos[first + t, c]. */
void oracle_embed(const uint32_t* tokens, int count, const float* token_table,
                  const float* position_table, int first_position, int width,
                  double* out);

/* Core/Utils/Half.cpp:8-78 semantics: fp32 -> fp16 round to nearest even
 * (including subnormals, infinities and NaN), and exact widening. bf16 the
 * same with an 8-bit exponent. */
uint16_t oracle_f32_to_f16_bits(float value);
float oracle_f16_bits_to_f32(uint16_t bits);
uint16_t oracle_f32_to_bf16_bits(float value);
float oracle_bf16_bits_to_f32(uint16_t bits);

/* std::mt19937 raw draws (Tests/Kernels/Common.h:75-88 relies on the
 * standard fixing this sequence). */
void oracle_mt19937_fill(uint32_t seed, int64_t count, uint32_t* out);

/* ---- the whole decoder ---- */

/* Tests/Decoder/Common.h:360-468: full-prefix recompute from position 0.
 * hidden_out [count, width], logits_out [count, vocab], both double. */
int oracle_decode_full(const oracle_shape* shape, const float* const* tensors,
                       const float* encoder_rows, int encoder_row_count,
                       const int* tokens, int count, double* hidden_out,
                       double* logits_out);

/* The same decoder with a KV cache: begin projects the cross keys and values
 * once (Decoder/Decoder.cpp:121-146), each step appends count tokens at the
 * current position (Decoder/Decoder.cpp:270-308). Row for row it performs the
 * same double operations in the same order as oracle_decode_full, so the two
 * are bitwise equal. */
typedef struct oracle_session oracle_session;

oracle_session* oracle_session_create(const oracle_shape* shape,
                                      const float* const* tensors);
void oracle_session_destroy(oracle_session* session);

/* rows = 0 means shape->cross_positions; rows above it is an error (-1). */
int oracle_session_begin(oracle_session* session, const float* encoder_rows,
                         int rows);

/* Returns 0, or -1 when count <= 0 or the step would pass max_positions
 * (nothing is changed then: Decoder/Decoder.cpp:276-289). Either output may
 * be null. */
int oracle_session_step(oracle_session* session, const int* tokens, int count,
                        double* hidden_out, double* logits_out);

int oracle_session_position(const oracle_session* session);

/* Greedy decode in the shape of Whisper::decodeTranscript with an all-zero
 * mask and no end-of-text stop (Whisper/Whisper.cpp:1186-1213): one prompt
 * step over prompt_count tokens, argmax of its last row, then `steps - 1`
 * single-token steps each fed the previous argmax. Writes `steps` tokens.
 * margins_or_null receives each step's top-1 minus top-2 logit, so a near tie
 * is visible. last_logits_or_null receives the final step's logits row. */
int oracle_greedy(oracle_session* session, const int* prompt, int prompt_count,
                  int steps, const float* mask_or_null, int* tokens_out,
                  double* margins_or_null, double* last_logits_or_null);

/* ---- the encoder (the step before the path: Encoder/Encoder.cpp:82-111) ---- */

typedef struct oracle_encoder_shape
{
    int mel_bins;
    int width;
    int heads;
    int layers;
    int feed_forward_width;
    int input_frames;
} oracle_encoder_shape;

/* Canonical encoder tensor order: model-level tensors, then
 * ORACLE_ENC_TENSORS_PER_LAYER per layer (HF names model.encoder.*). */
enum
{
    ORACLE_ENC_CONV1_W = 0, /* [width, mel_bins, 3] */
    ORACLE_ENC_CONV1_B,     /* [width] */
    ORACLE_ENC_CONV2_W,     /* [width, width, 3] */
    ORACLE_ENC_CONV2_B,
    ORACLE_ENC_POSITIONS,   /* [>= positions, width] */
    ORACLE_ENC_FINAL_NORM_W,
    ORACLE_ENC_FINAL_NORM_B,
    ORACLE_ENC_MODEL_TENSORS
};

enum
{
    ORACLE_EL_ATTN_NORM_W = 0,
    ORACLE_EL_ATTN_NORM_B,
    ORACLE_EL_Q_W,
    ORACLE_EL_Q_B,
    ORACLE_EL_K_W,
    ORACLE_EL_V_W,
    ORACLE_EL_V_B,
    ORACLE_EL_O_W,
    ORACLE_EL_O_B,
    ORACLE_EL_FINAL_NORM_W,
    ORACLE_EL_FINAL_NORM_B,
    ORACLE_EL_FC1_W,
    ORACLE_EL_FC1_B,
    ORACLE_EL_FC2_W,
    ORACLE_EL_FC2_B,
    ORACLE_ENC_TENSORS_PER_LAYER
};

/* Kernels/Conv1d.h:121-124: (length + 2 padding - kernel) / stride + 1, with
 * kernel 3 and padding 1 (Encoder/EncoderShape.h:20-23). */
int oracle_conv1d_output_length(int input_length, int stride);

/* Tests/Encoder/Common.h:398-441: [output_channels, output_length] out of
 * [input_channels, input_length], both channel-major; weight [output_channels,
 * input_channels, 3]; padded taps are skipped. */
void oracle_conv1d(const double* input, int input_channels, int input_length,
                   const float* weight, const float* bias, int output_channels,
                   int stride, double* out);

/* Tests/Encoder/Common.h:596-688: the whole encoder over a band-major mel
 * [mel_bins, input_frames]; out receives [positions, width] row-major. */
int oracle_encode(const oracle_encoder_shape* shape, const float* const* tensors,
                  const float* mel, double* out);

/* ---- the mel front end (Mel/MelSpectrogram.h:12-25) ---- */

/* Tests/Mel/ScalarMel.h:14-134: periodic Hann window, numpy-"reflect" padding
 * of fft_length / 2 each side, |DFT|^2 of every hop_length-th window (the
 * textbook sum), the [mel_count, bin_count] filterbank, log10(max(x, 1e-10)),
 * then (max(v, peak - 8) + 4) / 4 over the whole spectrogram. out receives
 * [mel_count, frame_count] (band-major). */
int oracle_mel_spectrogram(const float* samples, int sample_count, const float* filters, int fft_length,
                           int hop_length, int frame_count, int mel_count, double* out);

#ifdef __cplusplus
}
#endif

#endif
