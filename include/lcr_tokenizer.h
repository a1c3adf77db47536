/*
 * lcr_tokenizer.h — C-ABI of the byte-level BPE tokenizer (the reference's
 * lcr::Tokenizer, src/tokenizer.h:23-91), for bindings in other languages.
 *
 * A tokenizer is built from a Hugging Face tokenizer.json with the Llama 3
 * split pretokenizer; construction fails (NULL, message in
 * lcr_last_error_message()) on any other model type or pattern, with the
 * reference's messages. Nothing here touches a GPU.
 *
 * Output buffers: a call writes at most `capacity` items and always stores
 * the full count in *count (or *length); when that exceeds the capacity it
 * returns LCR_ERR_ARGUMENT, and the caller retries with a larger buffer.
 */
#ifndef LCR_TOKENIZER_H_
#define LCR_TOKENIZER_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lcr_tokenizer lcr_tokenizer;

/* Tokenizer::from_file (src/tokenizer.h:25) */
lcr_tokenizer* lcr_tokenizer_create(const char* tokenizer_json_path);
/* Tokenizer::from_json_string (src/tokenizer.h:26); `json` need not be NUL-terminated */
lcr_tokenizer* lcr_tokenizer_create_from_json(const char* json, size_t length);
void lcr_tokenizer_destroy(lcr_tokenizer* tok);

/* Tokenizer::encode(text, add_bos, parse_special) (src/tokenizer.h:34-35) */
int lcr_tokenizer_encode(const lcr_tokenizer* tok, const char* text, size_t length, int add_bos,
                         int parse_special, int32_t* ids, size_t capacity, size_t* count);
/* Tokenizer::decode(ids, skip_special) (src/tokenizer.h:37-38); not NUL-terminated */
int lcr_tokenizer_decode(const lcr_tokenizer* tok, const int32_t* ids, size_t n, int skip_special,
                         char* text, size_t capacity, size_t* length);
/* Tokenizer::vocab_size, bos_id, token_to_id, is_special (src/tokenizer.h:44-49) */
int lcr_tokenizer_vocab_size(const lcr_tokenizer* tok);
int lcr_tokenizer_bos_id(const lcr_tokenizer* tok);
int lcr_tokenizer_token_to_id(const lcr_tokenizer* tok, const char* token, size_t length);
int lcr_tokenizer_is_special(const lcr_tokenizer* tok, int id);

/* Tokenizer::split_pretokens (src/tokenizer.h:53): the byte offset at which
 * each pretoken ends, in order */
int lcr_split_pretokens(const char* text, size_t length, size_t* ends, size_t capacity, size_t* count);

#ifdef __cplusplus
}
#endif

#endif /* LCR_TOKENIZER_H_ */
