/* rpg_text.h -- the text front-end of the engine on its own: BBPE tokenizer,
 * Qwen3 ChatML rendering and reply parsing, host CPU only (no GPU call).
 *
 * No reference counterpart as an ABI: the reference links these pieces into
 * its generate call (src/tokenizer.h, src/chat_template.h, src/tool_parser.h)
 * and exposes them only there. This header gives tests and hosts direct
 * access to the same functions that rpg_engine_generate uses. Conventions of
 * rpg_engine.h: handles >= 0, failures -1 / NULL with rpg_engine_last_error,
 * returned strings freed with rpg_engine_free.
 */
#ifndef RPG_TEXT_H
#define RPG_TEXT_H

#include <stdint.h>

#include "rpg_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Tokenizer of a GGUF (its tokenizer.ggml.* metadata; no tensors loaded). */
RPG_API int32_t rpg_text_tokenizer_load(const char* gguf_path);
RPG_API void rpg_text_tokenizer_free(int32_t tok);
/* Vocabulary size, or -1. */
RPG_API int32_t rpg_text_vocab_size(int32_t tok);

/* Encode len bytes of text (special tokens matched when parse_special != 0,
 * reference src/tokenizer.cc:303-338). Writes up to cap ids; returns the
 * number of ids (call again with a larger cap when it exceeds cap), -1 on
 * failure. */
RPG_API int64_t rpg_text_encode(int32_t tok, const char* text, int64_t len, int32_t parse_special, int32_t* out,
                                int64_t cap);

/* Decode n ids (special tokens dropped when skip_special != 0, reference
 * src/tokenizer.cc:340-372). *out_len receives the byte length (the text may
 * hold NUL bytes). */
RPG_API char* rpg_text_decode(int32_t tok, const int32_t* ids, int64_t n, int32_t skip_special, int64_t* out_len);

/* Byte lengths of the pre-tokenizer's pieces of len bytes of text (no special
 * tokens); returns the number of pieces (up to cap written), -1 on failure. */
RPG_API int64_t rpg_text_split(int32_t tok, const char* text, int64_t len, int64_t* piece_lens, int64_t cap);

/* The ChatML prompt of a request (its "messages", "tools" and
 * "enable_thinking"; the generation prompt always added), as
 * rpg_engine_generate renders it (reference src/chat_template.cc). */
RPG_API char* rpg_text_render_chatml(const char* request_json);

/* Parse of len bytes of a decoded reply (reference src/tool_parser.cc):
 * {"text": ..., "reasoning": ..., "tool_calls": [{"name": ..., "arguments_raw":
 * ..., "arguments": ... or null, "ok": bool}], "unterminated_think": bool,
 * "unterminated_tool_call": bool}. */
RPG_API char* rpg_text_parse_reply(const char* text, int64_t len);

/* Pre-tokenizer classes of n code points from `first`: out[i] bit 0 letter
 * (\p{L}), bit 1 number (\p{N}), bit 2 space (\s) -- Unicode 15.1, as the
 * reference classifies (src/unicode.h). Returns 0, or -1. */
RPG_API int32_t rpg_text_char_classes(uint32_t first, int64_t n, uint8_t* out);

/* Parse a JSON document and write it back: python != 0 in json.dumps style
 * (", " / ": "), else compact. The form tool definitions take in the prompt
 * (reference src/json.cc:285-455). */
RPG_API char* rpg_text_json_redump(const char* json, int32_t python);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RPG_TEXT_H */
