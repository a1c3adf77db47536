// Byte-level BPE tokenizer for Llama 3 checkpoints, read from tokenizer.json.
//
// Interface of the reference's Tokenizer (src/tokenizer.h:23-91): from_model_dir
// / from_file / from_json_string, encode(text, add_bos, parse_special),
// decode / decode_one, vocab_size, bos_id, token_to_id, id_to_token,
// is_special, and the split_pretokens / byte_level_encode / byte_level_decode
// stages on their own; the messages of its rejections are kept, since its
// tests match them.
//
// Encoding, as Hugging Face's tokenizers runs a Llama 3 tokenizer.json:
//  1. added tokens (<|begin_of_text|>, <|eot_id|>, ...) are matched
//     literally, longest first, when parse_special is set;
//  2. every other span is cut into pretokens by the Llama 3 split pattern
//         (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}|
//          ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
//     evaluated by a hand-written matcher over code points (alternatives in
//     order, each with the regex engine's greedy-then-backtrack result);
//     \p{L} and \p{N} come from unicode_classes.inc, \s is the White_Space
//     property, and a byte that is not valid UTF-8 is one character of none
//     of these classes;
//  3. each pretoken's bytes are mapped to the GPT-2 byte-level alphabet;
//  4. BPE: the pretoken starts as one symbol per byte-level character, and the
//     adjacent pair of lowest merge rank is merged until none is left (a
//     binary heap over pair positions, stale entries skipped); with the
//     model's ignore_merges, a pretoken that is already a vocabulary entry is
//     emitted whole.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace lcr {

class Tokenizer {
 public:
  static Tokenizer from_model_dir(const std::string& model_dir);
  static Tokenizer from_file(const std::string& tokenizer_json_path);
  static Tokenizer from_json_string(const std::string& text);

  // parse_special: added tokens written in the text encode as themselves (the
  // chat template relies on it). add_bos: the begin-of-text token first, as
  // the checkpoint's post-processor adds for a raw completion.
  std::vector<int> encode(const std::string& text, bool add_bos = false, bool parse_special = true) const;
  std::string decode(const std::vector<int>& ids, bool skip_special = false) const;
  // One token's bytes, for streaming (a token may end inside a UTF-8 sequence).
  std::string decode_one(int id, bool skip_special = false) const;

  int vocab_size() const { return static_cast<int>(pieces_.size()); }
  int bos_id() const { return bos_id_; }
  int token_to_id(const std::string& token) const;  // -1 when absent
  const std::string& id_to_token(int id) const;
  bool is_special(int id) const;

  static std::vector<std::string> split_pretokens(const std::string& text);
  static std::string byte_level_encode(const std::string& raw);
  static std::string byte_level_decode(const std::string& encoded);

 private:
  struct Merge {
    int rank;
    int result;
  };
  struct Added {
    std::string content;
    int id;
    bool special;
  };

  void load(const std::string& json_text);
  void encode_span(const std::string& text, size_t begin, size_t end, std::vector<int>* out) const;
  void bpe(const std::string& pretoken, std::vector<int>* out) const;
  static uint64_t pair_key(int left, int right) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(left)) << 32) | static_cast<uint32_t>(right);
  }

  std::vector<std::string> pieces_;                // by id ("" for unused ids)
  std::vector<uint8_t> kind_;                      // by id: 0 unused, 1 BPE piece, 2 added, 3 added special
  std::unordered_map<std::string, int> piece_id_;  // BPE vocabulary
  std::unordered_map<uint64_t, Merge> merges_;     // (left id, right id) -> rank, merged id
  std::vector<Added> added_;                       // longest content first
  bool added_first_byte_[256] = {};
  bool ignore_merges_ = false;
  int bos_id_ = -1;
};

}  // namespace lcr
