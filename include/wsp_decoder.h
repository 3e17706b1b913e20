/*
 * wsp_decoder.h — a C binding of the C++ decoder surface (include/whispereacp):
 * the stub a non-C++ caller (Python ctypes, cgo, N-API) binds to drive
 * WSP::Decoder, WSP::Argmax and the greedy loop. Every function returns a
 * wsp_hip.h status; the message is wsp_decoder_last_error(). Device pointers
 * are plain pointers into memory the caller allocated on the same device.
 *
 * Each call names the reference C++ entry point it exposes.
 */
#ifndef WSP_DECODER_H
#define WSP_DECODER_H

#include "wsp_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The host-side error class behind a non-zero status, mirroring the
 * reference's exceptions. */
enum
{
    WSP_KIND_NONE = 0,
    WSP_KIND_MODEL_ERROR = 1,      /* WSP::ModelError (Model/ModelError.h:16-20) */
    WSP_KIND_LOGIC_ERROR = 2,      /* std::logic_error */
    WSP_KIND_INVALID_ARGUMENT = 3, /* std::invalid_argument */
    WSP_KIND_RUNTIME_ERROR = 4     /* std::runtime_error (HIP) */
};

/* One tensor of a decoder file: its HuggingFace name, storage ("F32", "F16",
 * "BF16"), extents and host bytes (row-major, little-endian). */
typedef struct wsp_tensor_entry
{
    const char* name;
    const char* dtype;
    int rank;
    const long long* extents;
    const void* data;
} wsp_tensor_entry;

typedef struct wsp_decoder wsp_decoder;

/* DecoderWeights(file, shape, packing) + Decoder(shape).prepare(device)
 * (Decoder/DecoderWeights.cpp:151-178, Decoder/Decoder.cpp:194-227) +
 * Argmax::prepare(maxPositions, vocabularySize). packing: 0 Float, 1 ExactHalf.
 * stream is the hipStream_t every call records into. */
int wsp_decoder_create(const wsp_decoder_shape* shape, const wsp_tensor_entry* tensors, int count,
                       int packing, int device, void* stream, wsp_decoder** out);
void wsp_decoder_destroy(wsp_decoder* decoder);
const char* wsp_decoder_last_error(const wsp_decoder* decoder);
int wsp_decoder_last_error_kind(const wsp_decoder* decoder);

/* Decoder::beginSequence (Decoder/Decoder.h:75-78). encoder_rows: device f32
 * [cross_positions, width]. */
int wsp_decoder_begin_sequence(wsp_decoder* decoder, const float* encoder_rows, int cross_position_count);

/* Decoder::step (Decoder/Decoder.h:92-96). tokens: device uint32 [count];
 * logits: device f32 [count, vocabulary]. */
int wsp_decoder_step(wsp_decoder* decoder, const uint32_t* tokens, int count, float* logits);

/* A single-token step and its argmax under mask (device f32 or null), the
 * token written to argmax_slot (device uint32) — Decoder::step followed by
 * Argmax::encode (Whisper/Whisper.cpp:1186-1213), fused when possible. */
int wsp_decoder_step_and_sample(wsp_decoder* decoder, const uint32_t* token, float* logits,
                                const float* mask, uint32_t* argmax_slot);

int wsp_decoder_position(const wsp_decoder* decoder);
int wsp_decoder_cross_positions(const wsp_decoder* decoder);
/* Decoder::hiddenStates (Decoder/Decoder.h:111-115): device f32 rows. */
const float* wsp_decoder_hidden_states(const wsp_decoder* decoder);

/* Whether single-token steps take the fused launch (default 1 when the
 * weights' projections share one storage). */
int wsp_decoder_set_fused(wsp_decoder* decoder, int enabled);
int wsp_decoder_uses_fused(const wsp_decoder* decoder);

/* Whether fused single-token steps run as the one persistent launch (1) or
 * as the per-op sequence (0); see wsp_hip_step_persistent. */
int wsp_decoder_step_persistent(const wsp_decoder* decoder);

/* The persistent step's watchdog word (see wsp_hip_device_status). */
int wsp_decoder_device_status(wsp_decoder* decoder, int* status, int clear);

/* Sets the watchdog word (see wsp_hip_raise_device_status). */
int wsp_decoder_raise_device_status(wsp_decoder* decoder);

/* Argmax::encode (Kernels/Argmax.h:236-241) into out (device uint32 [rows]). */
int wsp_decoder_argmax(wsp_decoder* decoder, const float* logits, int rows, int row_length,
                       const float* mask, uint32_t* out);

/* The greedy loop of Whisper::decodeTranscript (Whisper/Whisper.cpp:1361-1443)
 * over encoder_rows (device), prompt (host ints), with masks on the device
 * (or null). end_of_text < 0 never stops early. Writes up to `capacity`
 * tokens to tokens_out (host) and the transcript's full token count to
 * *count_out; a transcript longer than `capacity` returns WSP_ERR_CAPACITY
 * (its first `capacity` tokens written). A step whose device-side hand-over
 * timed out (wsp_hip_device_status) ends the call with WSP_ERR_HIP, kind
 * runtime error, and clears the word. */
int wsp_decoder_greedy(wsp_decoder* decoder, const float* encoder_rows, int cross_position_count,
                       const int* prompt, int prompt_count, int maximum_tokens, int end_of_text,
                       const float* first_mask, const float* later_mask, int* tokens_out, int capacity,
                       int* count_out, double* decode_seconds);

/* ---- safetensors files (WSP::SafeTensors, Model/SafeTensors.h) -----------
 * A mapped safetensors file and the decoder built from one. A malformed file
 * is refused when it is opened, with the reason in the last error. */
typedef struct wsp_safetensors wsp_safetensors;
typedef struct wsp_batch_decoder wsp_batch_decoder;

/* SafeTensors::fromFile / fromBytes (the bytes are copied). On failure *out
 * still receives a handle whose last error says why (close it). */
int wsp_safetensors_open(const char* path, wsp_safetensors** out);
int wsp_safetensors_open_bytes(const void* bytes, size_t size, wsp_safetensors** out);
void wsp_safetensors_close(wsp_safetensors* file);
const char* wsp_safetensors_last_error(const wsp_safetensors* file);
int wsp_safetensors_count(const wsp_safetensors* file);

/* Tensor `index` in name order: its name, dtype ("F32", "BF16", ...), rank,
 * up to `capacity` extents and byte count. */
int wsp_safetensors_tensor(const wsp_safetensors* file, int index, const char** name, const char** dtype, int* rank,
                           long long* extents, int capacity, long long* byte_count);

/* SafeTensors::readFloats: F32/F16/BF16/F64 tensors as floats into out
 * (capacity floats). */
int wsp_safetensors_read_floats(wsp_safetensors* file, const char* name, float* out, long long capacity);

/* The value of __metadata__[key], or null. */
const char* wsp_safetensors_metadata(const wsp_safetensors* file, const char* key);

/* DecoderShape::fromConfig over a HuggingFace config.json
 * (Decoder/DecoderShape.cpp:7-17); cross_positions 0 takes
 * max_source_positions. The reason for a failure goes to error. */
int wsp_shape_from_config(const char* config_path, int cross_positions, wsp_decoder_shape* out, char* error,
                          int error_capacity);

/* Whisper::buildSuppressionMasks and the prompt's ids from a config.json
 * (Whisper/Whisper.cpp:202-254): first_mask / later_mask receive
 * vocabulary_size floats each (host memory; 1 = suppressed), the first step's
 * adding begin_suppress_tokens; start_token / end_token receive
 * decoder_start_token_id and eos_token_id (-1 when absent). Either pointer
 * pair may be null. A token past the vocabulary is refused. */
int wsp_decoding_from_config(const char* config_path, float* first_mask, float* later_mask, int capacity,
                             int* start_token, int* end_token, char* error, int error_capacity);

/* The special tokens of a HuggingFace tokenizer.json's added_tokens
 * (WSP::SpecialTokens; Tokenizer/SpecialTokens.h:16-44): -1 where the
 * vocabulary names none. english is the <|en|> language token. */
typedef struct wsp_special_tokens
{
    int end_of_text;
    int start_of_transcript;
    int start_of_previous;
    int start_of_language_model;
    int translate;
    int transcribe;
    int no_timestamps;
    int no_speech;
    int first_timestamp;
    int timestamp_count;
    float timestamp_interval;
    int language_count;
    int english;
} wsp_special_tokens;

int wsp_special_tokens_from_file(const char* tokenizer_path, wsp_special_tokens* out, char* error,
                                 int error_capacity);

/* Whisper::buildPrompt (Whisper/Whisper.cpp:202-225): the English-only
 * prompt [start, <|notimestamps|>] from a config.json (decoder_start_token_id,
 * else the vocabulary's <|startoftranscript|>) and a tokenizer.json. Writes up
 * to `capacity` ids to prompt_out and their count to *count_out; a vocabulary
 * that names no <|notimestamps|>, or neither file a start token, is refused
 * with the reason in error. */
int wsp_prompt_from_files(const char* config_path, const char* tokenizer_path, int* prompt_out, int capacity,
                          int* count_out, char* error, int error_capacity);

/* ---- the tokenizer (Tokenizer/Tokenizer.h:27-80) --------------------------
 * Whisper's byte-level BPE from a tokenizer.json: host code. Every added token
 * is special (skipped by decode unless keep_special). Errors are negative
 * codes with the reason in `error` (open) or WSP_ERR_CAPACITY when an output
 * does not fit, with the needed count or length still reported. */
typedef struct wsp_tokenizer wsp_tokenizer;

int wsp_tokenizer_open(const char* path, wsp_tokenizer** out, char* error, int error_capacity);
int wsp_tokenizer_open_bytes(const char* json, size_t length, wsp_tokenizer** out, char* error, int error_capacity);
void wsp_tokenizer_close(wsp_tokenizer* tokenizer);
int wsp_tokenizer_size(const wsp_tokenizer* tokenizer);
int wsp_tokenizer_is_special(const wsp_tokenizer* tokenizer, int token);
/* The id of a token spelled `text` in the vocabulary's printable alphabet
 * (e.g. "\xc4\xa0the"), or -1. */
int wsp_tokenizer_token_for_text(const wsp_tokenizer* tokenizer, const char* text, size_t length);
/* Tokenizer::encode: UTF-8 (or any bytes) in, ids out; *count_out is the full
 * count even when it exceeds capacity (then WSP_ERR_CAPACITY). A host
 * allocation failure or a count past INT_MAX is WSP_ERR_CAPACITY, any other
 * tokenizer exception WSP_ERR_ARGUMENT; nothing escapes the call. */
int wsp_tokenizer_encode(const wsp_tokenizer* tokenizer, const char* text, size_t length, int* ids_out, int capacity,
                         int* count_out);
/* Tokenizer::decode / decodeKeepingSpecialTokens: the bytes and a NUL in
 * text_out; *length_out is the byte count without the NUL. Errors as for
 * wsp_tokenizer_encode. */
int wsp_tokenizer_decode(const wsp_tokenizer* tokenizer, const int* ids, int count, int keep_special, char* text_out,
                         int capacity, int* length_out);

/* wsp_decoder_create / wsp_batch_decoder_create over the tensors of a
 * safetensors file (mapped while the weights upload). */
int wsp_decoder_create_from_file(const char* path, const wsp_decoder_shape* shape, int packing, int device,
                                 void* stream, wsp_decoder** out);
int wsp_batch_decoder_create_from_file(const char* path, const wsp_decoder_shape* shape, int packing, int streams,
                                       int max_step_tokens, int device, void* stream, wsp_batch_decoder** out);

/* ---- independent streams decoded together (WSP::BatchedDecoder) ----------
 * No reference counterpart: `streams` sequences share one weight read per
 * step, each with its own caches; see wsp_batch_create in wsp_hip.h. The
 * file's projections and logits must share one 16-bit storage (F16/BF16). */

int wsp_batch_decoder_create(const wsp_decoder_shape* shape, const wsp_tensor_entry* tensors, int count,
                             int packing, int streams, int max_step_tokens, int device, void* stream,
                             wsp_batch_decoder** out);
void wsp_batch_decoder_destroy(wsp_batch_decoder* decoder);
const char* wsp_batch_decoder_last_error(const wsp_batch_decoder* decoder);
int wsp_batch_decoder_last_error_kind(const wsp_batch_decoder* decoder);

/* Decoder::beginSequence for every stream; encoder_rows: device f32
 * [streams][cross_position_count (0: all)][width]. */
int wsp_batch_decoder_begin(wsp_batch_decoder* decoder, const float* encoder_rows, int cross_position_count);

/* Decoder::step for every stream: tokens device uint32 [streams][count],
 * logits device f32 [streams·count][vocabulary]. With argmax_slots non-null
 * each stream's masked argmax of its last row lands in argmax_slots[s]. */
int wsp_batch_decoder_step(wsp_batch_decoder* decoder, const uint32_t* tokens, int count, float* logits,
                           const float* mask, uint32_t* argmax_slots);

/* One graph-replayed single-token step per stream over a token ring
 * [max_positions + 1][streams] (see wsp_batch_ring_step in wsp_hip.h). */
int wsp_batch_decoder_ring_step(wsp_batch_decoder* decoder, uint32_t* ring, float* logits, const float* mask);

int wsp_batch_decoder_position(const wsp_batch_decoder* decoder);
/* wsp_batch_product_storage (wsp_hip.h) of the decoder's batch; no reference
 * counterpart. */
int wsp_batch_decoder_product_storage(const wsp_batch_decoder* decoder);
const float* wsp_batch_decoder_hidden_states(const wsp_batch_decoder* decoder);

/* ---- Whisper end to end (Whisper/Whisper.h:144-560, the kernels backend) --
 * load parses config.json, preprocessor_config.json and tokenizer.json and
 * maps model.safetensors (no GPU work); it builds the prompt and the two
 * suppression masks. prepare uploads everything and sizes every
 * intermediate on `device`, ordered on `stream`; transcribe allocates
 * nothing. Errors are statuses with the reason in wsp_whisper_last_error:
 * WSP_ERR_SHAPE for a ModelError, WSP_ERR_CAPACITY for an output that does
 * not fit (the needed count still reported), WSP_ERR_LOGIC for a misuse. */
typedef struct wsp_whisper wsp_whisper;

int wsp_whisper_create(wsp_whisper** out);
void wsp_whisper_destroy(wsp_whisper* whisper);
const char* wsp_whisper_last_error(const wsp_whisper* whisper);
int wsp_whisper_last_error_kind(const wsp_whisper* whisper);
/* Whisper::load(directory): a missing file is refused naming it. */
int wsp_whisper_load(wsp_whisper* whisper, const char* model_directory);
/* Whisper::load(ModelFiles): the three JSON documents as NUL-terminated text
 * and the weights as a safetensors file path. */
int wsp_whisper_load_files(wsp_whisper* whisper, const char* config_json, const char* preprocessor_json,
                           const char* tokenizer_json, const char* weights_path);
/* Whisper::setPacksWeights, before prepare (1 = fp16 wherever exact, the default). */
int wsp_whisper_set_packs_weights(wsp_whisper* whisper, int pack);
int wsp_whisper_prepare(wsp_whisper* whisper, int device, void* stream);
/* Whisper::prompt(): up to `capacity` ids; *count_out is the full count. */
int wsp_whisper_prompt(wsp_whisper* whisper, int* tokens_out, int capacity, int* count_out);
/* firstStepMask() / laterStepMask(): vocabulary_size floats each (host),
 * nonzero = suppressed; either pointer may be null. */
int wsp_whisper_masks(wsp_whisper* whisper, float* first_mask, float* later_mask, int capacity);
int wsp_whisper_end_of_text(wsp_whisper* whisper, int* token_out);
int wsp_whisper_set_maximum_tokens(wsp_whisper* whisper, int count);
int wsp_whisper_maximum_tokens(wsp_whisper* whisper, int* count_out);
/* Whisper::setAudioContext: 0 (the whole window) or 1..positions. */
int wsp_whisper_set_audio_context(wsp_whisper* whisper, int positions);
int wsp_whisper_audio_context_for_samples(wsp_whisper* whisper, int sample_count, double margin_seconds,
                                          int* positions_out);
/* Whisper::transcribe: at most one window of samples (host memory), the
 * transcript's tokens (end-of-text excluded) to tokens_out. */
int wsp_whisper_transcribe(wsp_whisper* whisper, const float* samples, int sample_count, int* tokens_out,
                           int capacity, int* count_out);
/* Whisper::textForTokens: the bytes and a NUL in text_out. */
int wsp_whisper_text_for_tokens(wsp_whisper* whisper, const int* tokens, int count, char* text_out, int capacity,
                                int* length_out);
/* lastEncodeSeconds, lastDecodeSeconds, lastStepCount; any pointer may be null. */
int wsp_whisper_timing(wsp_whisper* whisper, double* encode_seconds, double* decode_seconds, int* steps);
/* The last run's encoded rows (device, [positions, width]). */
int wsp_whisper_encoded_rows(wsp_whisper* whisper, const float** rows_out, int* positions_out, int* width_out);

#ifdef __cplusplus
}
#endif

#endif
