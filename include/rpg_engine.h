/* rpg_engine.h -- C ABI of the MI355X (gfx950) Qwen3 engine.
 *
 * Drop-in replacement for the reference library's 10-function interface
 * (reference include/rpg_engine.h:52-117, implemented in src/engine.cc:195-549):
 * same names, argument meaning and error behaviour, so a host that binds the
 * reference (Unity P/Invoke, Python ctypes) binds this library unchanged.
 *
 * Conventions kept from the reference:
 *  - handles are int32, >= 0 valid, < 0 failure; monotonically increasing
 *    from 1 and never reused (reference src/engine.cc:90-91,232-234,305-307);
 *  - no exception crosses the ABI: failures return -1 / NULL and leave a
 *    thread-local message for rpg_engine_last_error (reference :175-191);
 *  - strings returned by generate / model_info are freed with rpg_engine_free;
 *  - one generate per session at a time; the registry lock covers lookup only.
 *
 * Token loop: prefill and decode run on the GPU (hand-written HIP kernels,
 * decode step captured as a hipGraph, on-GPU exact sampler).
 *
 * Text front-end (host CPU, around the GPU token loop): a request's
 * "messages" / "tools" / "enable_thinking" render as Qwen3 ChatML, tokenize
 * with the model's BBPE vocabulary, and the reply decodes and parses into
 * "text" and "tool_calls" as in the reference (src/engine.cc:366-515).
 *
 * Request extension: "input_ids": [int, ...] (with no "messages") supplies
 * prompt token ids directly; its response carries "output_ids" next to the
 * reference's four keys.
 */
#ifndef RPG_ENGINE_H
#define RPG_ENGINE_H

#include <stdint.h>

#if defined(__GNUC__)
#define RPG_API __attribute__((visibility("default")))
#else
#define RPG_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define RPG_ENGINE_OK 0

/* Engine version string (reference include/rpg_engine.h:52-53). */
RPG_API const char* rpg_engine_version(void);

/* Last error of this thread; not freed, overwritten by the next call
 * (reference include/rpg_engine.h:55-56). */
RPG_API const char* rpg_engine_last_error(void);

/* Load a GGUF; config_json may be NULL: {"max_pos": 4096, "max_seq": 0,
 * "threads": ignored}. Returns a model handle or -1
 * (reference include/rpg_engine.h:60-65, src/engine.cc:201-244). */
RPG_API int32_t rpg_engine_load_model(const char* model_path, const char* config_json);

/* Unload and destroy its sessions; invalid handle is a no-op
 * (reference include/rpg_engine.h:67-68, src/engine.cc:246-257). */
RPG_API void rpg_engine_unload_model(int32_t model);

/* New session with its own KV cache; session_json may be NULL: {"max_seq",
 * "max_tokens", "stop", "temperature", "seed"}
 * (reference include/rpg_engine.h:72-75, src/engine.cc:259-319). */
RPG_API int32_t rpg_engine_session_create(int32_t model, const char* session_json);

/* Destroy a session and free its KV cache (reference include/rpg_engine.h:77-78). */
RPG_API void rpg_engine_session_destroy(int32_t session);

/* Clear the session's cache and history, keep its memory and handle
 * (reference include/rpg_engine.h:80-81, src/engine.cc:337-347). */
RPG_API int32_t rpg_engine_session_reset(int32_t session);

/* Run one generation; UTF-8 JSON in and out (reference
 * include/rpg_engine.h:85-110, src/engine.cc:349-515). Response:
 * {"text", "tool_calls", "finish_reason", "usage", "output_ids"}. */
RPG_API char* rpg_engine_generate(int32_t session, const char* request_json);

/* Free a string returned by the engine (reference include/rpg_engine.h:112-113). */
RPG_API void rpg_engine_free(char* buf);

/* Model metadata JSON; free with rpg_engine_free (reference
 * include/rpg_engine.h:115-117, src/engine.cc:519-547). */
RPG_API char* rpg_engine_model_info(int32_t model);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RPG_ENGINE_H */
