/*
 * wsp_hip.h — the C ABI of the MI355X (gfx950) decoder kernels.
 *
 * Plain C: device pointers, sizes and status codes; no exceptions cross it and
 * no C++ or torch types appear in it. Every call is asynchronous and ordered
 * on the stream the context was created with; a context is bound to one
 * device and is not thread-safe. All workspaces are sized when the context is
 * created, so no call below allocates device memory.
 *
 * Each entry point names the reference interface it stands in for; the
 * C++ layer in include/whispereacp/ (Net, HipNet, Decoder, Argmax) calls these
 * exactly where the reference's KernelNet dispatched eacp programs.
 */
#ifndef WSP_HIP_H
#define WSP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Negative values map back onto the reference's exceptions in
 * the C++ layer: SHAPE/CAPACITY -> ModelError or std::invalid_argument,
 * LOGIC -> std::logic_error, HIP -> std::runtime_error. */
enum
{
    WSP_OK = 0,
    WSP_ERR_ARGUMENT = -1, /* a null pointer or a non-positive extent */
    WSP_ERR_SHAPE = -2,    /* extents that do not fit together */
    WSP_ERR_CAPACITY = -3, /* beyond what the context was sized for */
    WSP_ERR_HIP = -4,      /* the HIP runtime reported an error */
    WSP_ERR_LOGIC = -5,    /* misuse (e.g. unsupported head width) */
    WSP_ERR_DEVICE = -6    /* a device-side watchdog tripped */
};

/* Storage of a weight matrix. F32 is read as is; F16 and BF16 are widened to
 * float on load (Kernels/Linear.h:229-246 reads fp16 the same way). */
enum
{
    WSP_F32 = 0,
    WSP_F16 = 1,
    WSP_BF16 = 2
};

/* Projection epilogue flags (Kernels/Linear.h:213-227): GELU applies the exact
 * activation to x·Wᵀ + b; RESIDUAL adds the result into what y holds. */
enum
{
    WSP_LINEAR_GELU = 1,
    WSP_LINEAR_RESIDUAL = 2
};

/* Decoder/DecoderShape.h:20-83 */
typedef struct wsp_decoder_shape
{
    int width;
    int heads;
    int layers;
    int feed_forward_width;
    int vocabulary_size;
    int max_positions;
    int cross_positions;
} wsp_decoder_shape;

typedef struct wsp_hip_ctx wsp_hip_ctx;

/* Binds a context to `device` and `stream` (a hipStream_t; null is the
 * default stream) and sizes its workspaces for `shape` (attention partials,
 * argmax candidates). Replaces KernelNet::prepare's scratch and the
 * SingleQueryAttention/Argmax prepare() sizing (Net/KernelNet.cpp:133-207,
 * Kernels/SingleQueryAttention.cpp:32-60, Kernels/Argmax.cpp:26-40). */
int wsp_hip_ctx_create(const wsp_decoder_shape* shape, int device, void* stream,
                       wsp_hip_ctx** out);
void wsp_hip_ctx_destroy(wsp_hip_ctx* ctx);

/* The message behind the last non-zero status on this context. */
const char* wsp_hip_last_error(const wsp_hip_ctx* ctx);

/* The stream the context launches on (a hipStream_t). */
void* wsp_hip_stream(const wsp_hip_ctx* ctx);

/* y[r, o] = act(Σ_k x[r,k]·W[o,k] + b[o]) (+ y[r,o] when RESIDUAL).
 * x [rows, inner] f32, W [out, inner] row-major in `wdtype`, bias [out] f32 or
 * null (zero, which replaces the zero-bias buffers at
 * Net/KernelNet.cpp:440-458), y [rows, out] f32. Rows up to 16 take the split
 * GEMV, more take the tiled product. Replaces KernelNet::dispatchProjection
 * (Net/KernelNet.cpp:817-859) over SplitLinear / HalfWeightSplitLinear
 * (Kernels/Linear.h:129-276) and LinearProduct (Kernels/SimdTiledMatMul.h:470-486). */
int wsp_hip_linear(wsp_hip_ctx* ctx, const float* x, int rows, int inner, const void* weight,
                   int wdtype, const float* bias, float* y, int out, int flags);

/* y = (x - mean) * rsqrt(var + eps) * gamma + beta over rows of `width`
 * (biased variance of the centred values). Replaces LayerNorm
 * (Kernels/LayerNorm.h:19-90). */
int wsp_hip_layernorm(wsp_hip_ctx* ctx, const float* x, const float* gamma, const float* beta,
                      float* y, int rows, int width, float eps);

/* y[t, c] = token_table[tokens[t], c] + position_table[first + t, c].
 * Replaces Embed (Kernels/Embed.h:38-62). */
int wsp_hip_embed(wsp_hip_ctx* ctx, const uint32_t* tokens, int count, const float* token_table,
                  const float* position_table, int first_position, float* y, int width);

/* Multi-head attention of q_count queries (the last q_count of k_count
 * positions when causal) against k_count cached keys and values, heads of
 * width / heads columns. scale multiplies the summed dot product. One query
 * takes the split-key form (Kernels/SingleQueryAttention.h:505-556); several
 * take the causal multi-query form with the mask semantics of
 * Kernels/Attention.h:34-47. Replaces KernelNet::runCachedAttention
 * (Net/KernelNet.cpp:951-1013). Head width must be a multiple of 4, at most 64
 * (the reference's own limit, Kernels/SingleQueryAttention.cpp:32-45). */
int wsp_hip_attention(wsp_hip_ctx* ctx, const float* q, int q_count, const float* keys,
                      const float* values, int k_count, int width, int heads, int causal,
                      float scale, float* out);

/* wsp_hip_attention without a context, allocating nothing: the same kernels
 * and results, ordered on `stream` (a hipStream_t, null for the default
 * stream) on the caller's current device. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The split-key
 * partials live in a fixed device array of 2^20 floats (4 MiB) per GPU, held
 * until the process ends; a call whose partials exceed it returns
 * WSP_ERR_CAPACITY. Calls that overlap on one GPU share that array and race;
 * calls ordered on one stream do not. The reason for a non-zero status goes to
 * error (error_capacity bytes, may be null). */
int wsp_hip_attention_static(const float* q, int q_count, const float* keys, const float* values,
                             int k_count, int width, int heads, int causal, float scale, float* out,
                             void* stream, char* error, int error_capacity);

/* out[r] = the first j maximising logits[r * row_length + j] over the j with
 * mask[j] == 0 (mask may be null); all suppressed gives 0. Replaces Argmax
 * (Kernels/Argmax.h:46-262, Kernels/Argmax.cpp:43-81). */
int wsp_hip_argmax(wsp_hip_ctx* ctx, const float* logits, int rows, int row_length,
                   const float* mask, uint32_t* out);

/* K = X·Wkᵀ and V = X·Wvᵀ + bv for `rows` encoder rows of `width`, with fp32
 * accumulation; Wk, Wv [width, width] in `wdtype`. Replaces the two
 * appendLinear calls per layer of recordSequenceStart
 * (Decoder/Decoder.cpp:121-146) that route to LinearProduct. */
int wsp_hip_project_cross_kv(wsp_hip_ctx* ctx, const float* x, int rows, int width,
                             const void* wk, const void* wv, const float* bv, int wdtype,
                             float* k_out, float* v_out);

/* ---- the fused single-token step ----------------------------------------- */

/* Device pointers of one decoder layer's tensors (Decoder/DecoderWeights.h:25-63).
 * Projection weights are in the table's wdtype; everything else is f32. The
 * fused step reads q/k/v of each attention through one concatenated
 * [3·width, width] block: qkv_weight points at q_proj, followed by k_proj and
 * v_proj; qkv_bias is [q_bias | 0 | v_bias] (k_proj has no bias). */
typedef struct wsp_layer_tensors
{
    const float* self_norm_w;
    const float* self_norm_b;
    const void* self_qkv_w;
    const float* self_qkv_b;
    const void* self_out_w;
    const float* self_out_b;
    const float* cross_norm_w;
    const float* cross_norm_b;
    const void* cross_q_w;
    const float* cross_q_b;
    const void* cross_out_w;
    const float* cross_out_b;
    const float* final_norm_w;
    const float* final_norm_b;
    const void* fc1_w;
    const float* fc1_b;
    const void* fc2_w;
    const float* fc2_b;
    float* self_keys;    /* [max_positions, width] f32 */
    float* self_values;  /* [max_positions, width] f32 */
    const float* cross_keys;   /* [cross_positions, width] f32 */
    const float* cross_values; /* [cross_positions, width] f32 */
} wsp_layer_tensors;

typedef struct wsp_decoder_tensors
{
    int wdtype;                   /* storage of every projection weight */
    const float* token_embedding; /* [vocab, width] f32 (the gather's table) */
    const void* logits_weight;    /* [vocab, width] in logits_wdtype (tied) */
    int logits_wdtype;
    const float* position_embedding; /* [max_positions, width] f32 */
    const float* final_norm_w;
    const float* final_norm_b;
    const wsp_layer_tensors* layers; /* device-independent host array, `layers` long */
} wsp_decoder_tensors;

/* One single-token decoder step fused into one persistent launch: embeds
 * tokens[0] at `position`, runs every layer (appending the new key and value
 * rows to the self caches at row `position`), writes the final hidden row, the
 * logits row and — when argmax_out is non-null — the masked argmax into
 * *argmax_out. cross_rows encoder rows are attended. Same contract as
 * Decoder::step with one token (Decoder/Decoder.cpp:270-308) followed by
 * Argmax::encode (Whisper/Whisper.cpp:1164-1184). */
int wsp_hip_decoder_step(wsp_hip_ctx* ctx, const wsp_decoder_tensors* tensors,
                         const uint32_t* tokens, int position, int cross_rows, float* hidden,
                         float* logits, const float* mask, uint32_t* argmax_out);

/* A step of token_count tokens at position .. position + token_count - 1
 * (Decoder::step, Decoder/Decoder.cpp:270-308 with tokenCount tokens, and
 * the causal self attention of Kernels/Attention.h:34-47): token i sees the
 * keys of every token before it. hidden receives [token_count, width] and
 * logits [token_count, vocab]; with argmax_out non-null the masked argmax of
 * the last row lands there. On the persistent path a launch carries up to
 * four tokens (fewer where the shape leaves fewer head groups per token), so
 * their rows share each weight read; a step is as many launches as that
 * takes. Otherwise each token runs the per-op sequence. */
int wsp_hip_decoder_step_tokens(wsp_hip_ctx* ctx, const wsp_decoder_tensors* tensors,
                                const uint32_t* tokens, int token_count, int position, int cross_rows,
                                float* hidden, float* logits, const float* mask, uint32_t* argmax_out);

/* Whether wsp_hip_decoder_step runs as the one persistent launch on this
 * context (1) or falls back to the per-op sequence (0) because the shape or
 * device is outside the persistent kernel's capacities. No reference
 * counterpart: it reports which of this build's two step forms is in use. */
int wsp_hip_step_persistent(const wsp_hip_ctx* ctx);

/* Waits for the context's stream, then reports the persistent step's
 * watchdog word in *status: 0 when every hand-over completed, 1 when a wait
 * timed out and the launch left early (its outputs are then undefined).
 * clear != 0 resets the word. No reference counterpart: the reference's
 * passes cannot time out. */
int wsp_hip_device_status(wsp_hip_ctx* ctx, int* status, int clear);

/* Enqueues a copy of the watchdog word into *dst (host memory, pinned for the
 * copy to stay asynchronous) on the context's stream, so a caller reading a
 * step's outputs behind an event reads the word of the same point in the
 * stream. Writes 0 at once when the context runs no persistent step. No
 * reference counterpart (see wsp_hip_device_status). */
int wsp_hip_device_status_copy(wsp_hip_ctx* ctx, int* dst);

/* One launch that writes, ordered after the work already on the context's
 * stream, host_pair[0] = *slot (a sampled token, device memory) and
 * host_pair[1] = the watchdog word (0 when the context runs no persistent
 * step). host_pair is pinned host memory (hipHostMalloc). It replaces a token
 * copy and a wsp_hip_device_status_copy in a greedy loop that reads each
 * token behind an event: one small launch instead of two copies. No
 * reference counterpart (see wsp_hip_device_status). */
int wsp_hip_step_report(wsp_hip_ctx* ctx, const uint32_t* slot, int* host_pair);

/* Hands host_pair to the next sampling step (wsp_hip_decoder_step with
 * argmax_out) on this context: a persistent step writes the token and the
 * watchdog word there itself when its argmax fold ends, so the
 * wsp_hip_step_report(ctx, slot, host_pair) that follows it launches nothing.
 * A step that trips its watchdog writes nothing: the caller puts a nonzero
 * word in host_pair[1] beforehand and reads it as a trip. Other steps leave
 * the report to wsp_hip_step_report as before. No reference counterpart (see
 * wsp_hip_device_status). */
int wsp_hip_step_report_next(wsp_hip_ctx* ctx, int* host_pair);

/* Sets the watchdog word as a tripped wait does: later persistent steps on
 * this context leave at their first long wait, and every caller that reads
 * the word reports the failure, until it is cleared. No reference
 * counterpart: for a caller abandoning a context's work, and for tests of the
 * failure path, which then run without a real time-out. */
int wsp_hip_raise_device_status(wsp_hip_ctx* ctx);

/* ---- batched independent streams ------------------------------------------
 * No reference counterpart: the reference decodes one sequence per Decoder.
 * A batch holds `streams` independent sequences that share one weight read
 * per step. Each has its own self and cross caches, all advance together,
 * and every stream's rows equal what Decoder::step computes for that stream
 * alone (Decoder/Decoder.cpp:270-308). Projections need 16-bit storage (F16
 * or BF16): they run on the matrix cores with the fp32 activations split into
 * exact 16-bit parts. */

/* One layer's cross-attention key and value projections (Decoder/DecoderWeights.h:25-63). */
typedef struct wsp_cross_tensors
{
    const void* key_w;    /* [width, width], no bias (k_proj) */
    const void* value_w;  /* [width, width] */
    const float* value_b; /* [width] */
} wsp_cross_tensors;

typedef struct wsp_batch wsp_batch;

/* Allocates every stream's caches (self [layers][streams][max_positions][width],
 * cross [layers][cross_positions][streams][width] — key-major — f32), a
 * fragment-major copy of the projection and logits weights, and the step buffers
 * for up to max_step_tokens tokens per stream per step; streams ×
 * max_step_tokens ≤ 128. wdtype is the projections' storage (WSP_F16 or
 * WSP_BF16). Decoder::prepare's role (Decoder/Decoder.cpp:194-227), per stream. */
int wsp_batch_create(const wsp_decoder_shape* shape, int streams, int max_step_tokens, int wdtype, int device,
                     void* stream, wsp_batch** out);
void wsp_batch_destroy(wsp_batch* batch);
const char* wsp_batch_last_error(const wsp_batch* batch);
int wsp_batch_position(const wsp_batch* batch);
int wsp_batch_cross_rows(const wsp_batch* batch);

/* Decoder::beginSequence for every stream (Decoder/Decoder.cpp:241-268):
 * projects the cross keys and values of each stream's first cross_rows
 * encoder rows (0: all) and resets the position. encoder_rows: device f32
 * [streams][cross_rows][width]; layers: host array of `layers` entries. */
int wsp_batch_begin(wsp_batch* batch, const wsp_cross_tensors* layers, int wdtype, const float* encoder_rows,
                    int cross_rows);

/* Decoder::step for every stream: tokens is device uint32 [streams][count]
 * (stream-major), logits device f32 [streams·count][vocabulary], hidden
 * (device f32 [streams·count][width]) or null. With argmax_out non-null,
 * argmax_out[s] receives the masked argmax of stream s's last row
 * (Argmax::encode, Kernels/Argmax.h:236-241), so it can feed the next step.
 * The layer table's cache pointers are not used: the batch owns its caches.
 * The products read the batch's own fragment-major copy of the projection and
 * logits weights, packed on the batch's stream the first time a table is
 * passed (here or to wsp_batch_ring_step) and whenever its pointers change: a
 * table with the same pointers is taken to hold the same weights. */
int wsp_batch_step(wsp_batch* batch, const wsp_decoder_tensors* tensors, const uint32_t* tokens, int count,
                   float* hidden, float* logits, const float* mask, uint32_t* argmax_out);

/* No reference counterpart: the storage of the weight copy the products read,
 * after the last packed table. A bf16 table is packed as exact fp16 multiples
 * w·2^k per matrix (k puts the matrix's largest magnitude in fp16's top
 * binade; the products divide 2^k out of each sum) when every value of every
 * matrix narrows exactly, and the step then takes two fp16 parts of each
 * input instead of three bf16 ones: WSP_F16 then and for fp16 tables,
 * WSP_BF16 for a bf16 table that does not narrow, 0 before any table. */
int wsp_batch_product_storage(const wsp_batch* batch);

/* One single-token step for every stream driven by a token ring: ring is
 * device uint32 [max_positions + 1][streams], position-major. The step reads
 * each stream's token at the current position p from ring[p] and writes its
 * masked greedy successor to ring[p + 1]; logits [streams][vocabulary] are
 * written too. Nothing in it depends on p on the host, so it is captured once
 * as a HIP graph and replayed (re-captured when ring, logits, mask, the cross
 * rows or the weight table change). Needs p >= 1 (the prompt step runs
 * through wsp_batch_step, its argmax_out pointing at ring[p]). No reference
 * counterpart: Whisper::decodeTranscript's device-side token feedback
 * (Whisper/Whisper.cpp:1361-1443) for a batch, without per-launch host cost. */
int wsp_batch_ring_step(wsp_batch* batch, const wsp_decoder_tensors* tensors, uint32_t* ring, float* logits,
                        const float* mask);

/* Layer `layer`'s caches of stream 0; stream s starts max_positions·width
 * (self) floats later, key k of stream s of the cross caches sits at
 * (k·streams + s)·width. */
int wsp_batch_self_cache(const wsp_batch* batch, int layer, const float** keys, const float** values);
int wsp_batch_cross_cache(const wsp_batch* batch, int layer, const float** keys, const float** values);

/* ---------------------------------------------------------------------------
 * The encoder: the step before the decode path (Encoder/Encoder.h:8-71,
 * Encoder/Encoder.cpp:82-175). A mel [mel_bins, input_frames] band-major in,
 * [positions, width] rows out, positions = input_frames / 2 for Whisper's
 * stride-two second convolution (Encoder/EncoderShape.cpp:19-33).
 * ------------------------------------------------------------------------- */

/* Encoder/EncoderShape.h:25-67 */
typedef struct wsp_encoder_shape
{
    int mel_bins;
    int width;
    int heads;
    int layers;
    int feed_forward_width;
    int input_frames;
} wsp_encoder_shape;

/* Encoder/EncoderWeights.h:19-36, HuggingFace's model.encoder.layers.<i>.*
 * tensors: projections in `wdtype` storage, everything else fp32 (the
 * reference widens every non-projection tensor, Encoder/EncoderWeights.h:44-52).
 * k_proj has no bias. The *_scale fields are the power of two each stored
 * projection carries (wsp_encoder_scaled_halves: bf16 weights held as exact
 * fp16 multiples), in [2^-126, 2^126]; the products divide it out. 0 or 1:
 * stored as they are. */
typedef struct wsp_encoder_layer_tensors
{
    const float* attention_norm_w;
    const float* attention_norm_b;
    const void* q_w;
    const float* q_b;
    const void* k_w;
    const void* v_w;
    const float* v_b;
    const void* out_w;
    const float* out_b;
    const float* final_norm_w;
    const float* final_norm_b;
    const void* fc1_w;
    const float* fc1_b;
    const void* fc2_w;
    const float* fc2_b;
    float q_scale, k_scale, v_scale, out_scale, fc1_scale, fc2_scale;
} wsp_encoder_layer_tensors;

/* Encoder/EncoderWeights.h:70-93: conv1 [width, mel_bins, 3], conv2 [width,
 * width, 3] and their biases, embed_positions [>= positions, width] and the
 * final LayerNorm, all fp32. */
typedef struct wsp_encoder_tensors
{
    int wdtype; /* the projections' storage (WSP_F32, WSP_F16, WSP_BF16) */
    const float* conv1_w;
    const float* conv1_b;
    const float* conv2_w;
    const float* conv2_b;
    const float* positions;
    const float* final_norm_w;
    const float* final_norm_b;
    const wsp_encoder_layer_tensors* layers; /* host array, `layers` long */
} wsp_encoder_tensors;

typedef struct wsp_encoder wsp_encoder;

/* Encoder::prepare (Encoder/Encoder.cpp:113-146): every intermediate sized for
 * the shape's window, on `device`, ordered on `stream`. */
int wsp_encoder_create(const wsp_encoder_shape* shape, int device, void* stream, wsp_encoder** out);
void wsp_encoder_destroy(wsp_encoder* encoder);
const char* wsp_encoder_last_error(const wsp_encoder* encoder);

/* Encoder::encode (Encoder/Encoder.cpp:148-174): reads the first
 * min(2 * position_count, input_frames) frames of each band of `mel` (device,
 * [mel_bins, input_frames]) and writes position_count rows of width floats to
 * `output` (device); position_count 0 is the whole window. A count past the
 * window is WSP_ERR_SHAPE before anything is launched. No allocation. */
int wsp_encoder_encode(wsp_encoder* encoder, const wsp_encoder_tensors* tensors, const float* mel, float* output,
                       int position_count);

/* No reference counterpart: a storage choice of the loader, as the
 * reference's exact fp16 packing of F32 projections is
 * (Model/SafeTensors.cpp:554-592). A bf16 projection of `count` values
 * (host memory) written to `halves` (host memory) as fp16 values w·2^k, k
 * the largest shift that leaves every value finite, and *scale = 2^k. The
 * products then read two fp16 parts of their fp32 input instead of three
 * bf16 ones. WSP_OK when every value narrows exactly; WSP_ERR_LOGIC when one
 * does not (or is not finite): keep the bf16 storage then; WSP_ERR_SHAPE when
 * the shape's encoder does not take scaled projections (it needs its products
 * over pre-split inputs: width and ffn width multiples of 128, width at most
 * 2048). No GPU work. */
int wsp_encoder_scaled_halves(const wsp_encoder_shape* shape, const void* bf16, size_t count, void* halves,
                              float* scale);

/* ---------------------------------------------------------------------------
 * The mel front end (Mel/MelSpectrogram.h:12-25, Mel/MelShape.h:16-30): 30 s
 * of 16 kHz samples in, the [mel_count, frame_count] normalised log-mel the
 * encoder reads out. The filterbank ([mel_count, fft_length / 2 + 1],
 * preprocessor_config.json's matrix) is an argument of every call, as in the
 * reference.
 * ------------------------------------------------------------------------- */
typedef struct wsp_mel_shape
{
    int sample_count; /* 480000 */
    int fft_length;   /* 400 */
    int hop_length;   /* 160 */
    int frame_count;  /* 3000 */
    int mel_count;    /* 80 */
} wsp_mel_shape;

typedef struct wsp_mel wsp_mel;

/* MelSpectrogram::prepare: the window, the DFT basis and every intermediate. */
int wsp_mel_create(const wsp_mel_shape* shape, int device, void* stream, wsp_mel** out);
void wsp_mel_destroy(wsp_mel* mel);
const char* wsp_mel_last_error(const wsp_mel* mel);

/* MelSpectrogram::encode: samples [sample_count], filters [mel_count,
 * fft_length / 2 + 1] and output [mel_count, frame_count], all device
 * memory. No allocation. */
int wsp_mel_encode(wsp_mel* mel, const float* samples, const float* filters, float* output);

#ifdef __cplusplus
}
#endif

#endif
