// C-ABI of the tokenizer (include/lcr_tokenizer.h).
#include "../../include/lcr_tokenizer.h"

#include <algorithm>
#include <cstring>

#include "capi_util.h"
#include "tokenizer.h"

struct lcr_tokenizer {
  lcr::Tokenizer tok;
};

using lcr::capi::guarded;

namespace {

lcr_tokenizer* make(const std::string& json) {
  lcr::capi::clear_error();
  try {
    return new lcr_tokenizer{lcr::Tokenizer::from_json_string(json)};
  } catch (const std::exception& e) {
    lcr::capi::set_error(e.what());
    return nullptr;
  }
}

}  // namespace

extern "C" lcr_tokenizer* lcr_tokenizer_create(const char* path) {
  lcr::capi::clear_error();
  try {
    return new lcr_tokenizer{lcr::Tokenizer::from_file(path != nullptr ? path : "")};
  } catch (const std::exception& e) {
    lcr::capi::set_error(e.what());
    return nullptr;
  }
}

extern "C" lcr_tokenizer* lcr_tokenizer_create_from_json(const char* json, size_t length) {
  return make(std::string(json != nullptr ? json : "", json != nullptr ? length : 0));
}

extern "C" void lcr_tokenizer_destroy(lcr_tokenizer* tok) { delete tok; }

extern "C" int lcr_tokenizer_encode(const lcr_tokenizer* tok, const char* text, size_t length, int add_bos,
                                    int parse_special, int32_t* ids, size_t capacity, size_t* count) {
  lcr::capi::clear_error();
  CAPI_CHECK(tok != nullptr && count != nullptr, "encode needs a tokenizer and a count");
  return guarded([&] {
    const std::vector<int> out = tok->tok.encode(std::string(text != nullptr ? text : "", length), add_bos != 0,
                                                 parse_special != 0);
    *count = out.size();
    CAPI_CHECK(out.size() <= capacity, "encode produced " << out.size() << " ids for a buffer of " << capacity);
    std::copy(out.begin(), out.end(), ids);
    return LCR_OK;
  });
}

extern "C" int lcr_tokenizer_decode(const lcr_tokenizer* tok, const int32_t* ids, size_t n, int skip_special,
                                    char* text, size_t capacity, size_t* length) {
  lcr::capi::clear_error();
  CAPI_CHECK(tok != nullptr && length != nullptr, "decode needs a tokenizer and a length");
  return guarded([&] {
    const std::string out = tok->tok.decode(std::vector<int>(ids, ids + n), skip_special != 0);
    *length = out.size();
    CAPI_CHECK(out.size() <= capacity, "decode produced " << out.size() << " bytes for a buffer of " << capacity);
    std::memcpy(text, out.data(), out.size());
    return LCR_OK;
  });
}

extern "C" int lcr_tokenizer_vocab_size(const lcr_tokenizer* tok) { return tok != nullptr ? tok->tok.vocab_size() : -1; }
extern "C" int lcr_tokenizer_bos_id(const lcr_tokenizer* tok) { return tok != nullptr ? tok->tok.bos_id() : -1; }

extern "C" int lcr_tokenizer_token_to_id(const lcr_tokenizer* tok, const char* token, size_t length) {
  return tok != nullptr ? tok->tok.token_to_id(std::string(token, length)) : -1;
}

extern "C" int lcr_tokenizer_is_special(const lcr_tokenizer* tok, int id) {
  return tok != nullptr && tok->tok.is_special(id) ? 1 : 0;
}

extern "C" int lcr_split_pretokens(const char* text, size_t length, size_t* ends, size_t capacity, size_t* count) {
  lcr::capi::clear_error();
  CAPI_CHECK(count != nullptr, "split needs a count");
  return guarded([&] {
    const std::vector<std::string> pieces = lcr::Tokenizer::split_pretokens(std::string(text, length));
    *count = pieces.size();
    CAPI_CHECK(pieces.size() <= capacity, "split produced " << pieces.size() << " pieces for " << capacity);
    size_t end = 0;
    for (size_t i = 0; i < pieces.size(); ++i) {
      end += pieces[i].size();
      ends[i] = end;
    }
    return LCR_OK;
  });
}
