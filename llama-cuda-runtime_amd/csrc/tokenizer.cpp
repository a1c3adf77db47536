#include "tokenizer.h"

#include <algorithm>
#include <fstream>
#include <queue>
#include <sstream>

#include "json.h"

namespace lcr {
namespace {

struct CodeRange {
  uint32_t lo, hi;
};
#include "unicode_classes.inc"

// One character of the text as the split pattern sees it.
enum CharClass : uint8_t { kOther, kLetter, kNumber, kSpace };
constexpr uint32_t kInvalidByte = 0xFFFFFFFFu;  // a byte that is not valid UTF-8

template <size_t N>
bool in_ranges(const CodeRange (&r)[N], uint32_t cp) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < r[mid].lo) {
      hi = mid;
    } else if (cp > r[mid].hi) {
      lo = mid + 1;
    } else {
      return true;
    }
  }
  return false;
}

// The Unicode White_Space property (the regex engine's \s).
bool is_white_space(uint32_t cp) {
  if (cp <= 0x20) return cp == 0x20 || (cp >= 0x09 && cp <= 0x0D);
  switch (cp) {
    case 0x85: case 0xA0: case 0x1680: case 0x2028: case 0x2029: case 0x202F: case 0x205F: case 0x3000:
      return true;
    default:
      return cp >= 0x2000 && cp <= 0x200A;
  }
}

CharClass classify(uint32_t cp) {
  if (cp == kInvalidByte) return kOther;
  if (cp < 0x80) {
    if ((cp | 0x20) >= 'a' && (cp | 0x20) <= 'z') return kLetter;
    if (cp >= '0' && cp <= '9') return kNumber;
    return is_white_space(cp) ? kSpace : kOther;
  }
  if (is_white_space(cp)) return kSpace;
  if (in_ranges(kLetterRanges, cp)) return kLetter;
  if (in_ranges(kNumberRanges, cp)) return kNumber;
  return kOther;
}

// Decodes the code point at s[i]; a malformed or truncated sequence yields
// kInvalidByte for its first byte alone.
uint32_t next_code_point(const std::string& s, size_t i, size_t* len) {
  const auto b = [&](size_t k) { return static_cast<unsigned char>(s[k]); };
  const unsigned char c0 = b(i);
  if (c0 < 0x80) {
    *len = 1;
    return c0;
  }
  int n = 0;
  uint32_t cp = 0;
  if ((c0 & 0xE0) == 0xC0) {
    n = 2;
    cp = c0 & 0x1F;
  } else if ((c0 & 0xF0) == 0xE0) {
    n = 3;
    cp = c0 & 0x0F;
  } else if ((c0 & 0xF8) == 0xF0) {
    n = 4;
    cp = c0 & 0x07;
  }
  if (n == 0 || i + n > s.size()) {
    *len = 1;
    return kInvalidByte;
  }
  for (int k = 1; k < n; ++k) {
    if ((b(i + k) & 0xC0) != 0x80) {
      *len = 1;
      return kInvalidByte;
    }
    cp = (cp << 6) | (b(i + k) & 0x3F);
  }
  static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
  if (cp < kMin[n] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) {
    *len = 1;
    return kInvalidByte;
  }
  *len = static_cast<size_t>(n);
  return cp;
}

void append_utf8(std::string* out, uint32_t cp) {
  if (cp < 0x80) {
    out->push_back(static_cast<char>(cp));
  } else if (cp < 0x800) {
    out->push_back(static_cast<char>(0xC0 | (cp >> 6)));
    out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
  } else if (cp < 0x10000) {
    out->push_back(static_cast<char>(0xE0 | (cp >> 12)));
    out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
    out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
  } else {
    out->push_back(static_cast<char>(0xF0 | (cp >> 18)));
    out->push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
    out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
    out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
  }
}

// The GPT-2 byte-level alphabet: the printable bytes '!'..'~', 0xA1..0xAC and
// 0xAE..0xFF stand for themselves; the other 68 bytes take the code points
// 256, 257, ... in byte order.
struct ByteAlphabet {
  uint32_t to_cp[256];
  std::unordered_map<uint32_t, unsigned char> to_byte;
  ByteAlphabet() {
    uint32_t extra = 256;
    for (int b = 0; b < 256; ++b) {
      const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE);
      to_cp[b] = printable ? static_cast<uint32_t>(b) : extra++;
      to_byte[to_cp[b]] = static_cast<unsigned char>(b);
    }
  }
};

const ByteAlphabet& alphabet() {
  static const ByteAlphabet a;
  return a;
}

// The Llama 3 split pattern as tokenizer.json writes it (after JSON decoding).
const char* const kLlama3Pattern =
    "(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\\r\\n\\p{L}\\p{N}]?\\p{L}+|\\p{N}{1,3}| ?[^\\s\\p{L}\\p{N}]+[\\r\\n]*|"
    "\\s*[\\r\\n]+|\\s+(?!\\S)|\\s+";

// Code points of a span with their byte offsets and classes.
struct Chars {
  std::vector<uint32_t> cp;
  std::vector<size_t> at;  // byte offset; at[n] = end
  std::vector<CharClass> cls;
  explicit Chars(const std::string& text) {
    size_t i = 0;
    while (i < text.size()) {
      size_t len = 1;
      const uint32_t c = next_code_point(text, i, &len);
      cp.push_back(c);
      at.push_back(i);
      cls.push_back(classify(c));
      i += len;
    }
    at.push_back(text.size());
  }
  size_t size() const { return cp.size(); }
  bool is_crlf(size_t i) const { return cp[i] == '\r' || cp[i] == '\n'; }
  size_t run(size_t i, CharClass c) const {
    size_t j = i;
    while (j < size() && cls[j] == c) ++j;
    return j;
  }
};

char ascii_lower(uint32_t cp) { return cp < 0x80 ? static_cast<char>(cp | 0x20) : '\0'; }

// Length in code points of the pattern's match at i (alternatives in order).
size_t match_at(const Chars& t, size_t i) {
  const size_t n = t.size();
  // (?i:'s|'t|'re|'ve|'m|'ll|'d)
  if (t.cp[i] == '\'' && i + 1 < n) {
    const char a = ascii_lower(t.cp[i + 1]);
    if (a == 's' || a == 't' || a == 'm' || a == 'd') return 2;
    if (i + 2 < n) {
      const char b = ascii_lower(t.cp[i + 2]);
      if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return 3;
    }
  }
  // [^\r\n\p{L}\p{N}]?\p{L}+
  if (t.cls[i] == kLetter) return t.run(i, kLetter) - i;
  if (t.cls[i] != kNumber && !t.is_crlf(i) && i + 1 < n && t.cls[i + 1] == kLetter) {
    return t.run(i + 1, kLetter) - i;
  }
  // \p{N}{1,3}
  if (t.cls[i] == kNumber) return std::min<size_t>(3, t.run(i, kNumber) - i);
  // ' ?[^\s\p{L}\p{N}]+[\r\n]*'
  size_t j = i;
  if (t.cp[i] == ' ' && i + 1 < n && t.cls[i + 1] == kOther) j = i + 1;
  if (t.cls[j] == kOther) {
    size_t e = t.run(j, kOther);
    while (e < n && t.is_crlf(e)) ++e;
    return e - i;
  }
  // The rest start with white space.
  const size_t e = t.run(i, kSpace);
  // \s*[\r\n]+ : up to and including the run's last line break
  for (size_t k = e; k > i; --k) {
    if (t.is_crlf(k - 1)) return k - i;
  }
  // \s+(?!\S) : the whole run at the end of the text, else all but its last
  if (e == n) return e - i;
  if (e - i >= 2) return e - i - 1;
  // \s+
  return e - i;
}

std::string read_file(const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  LCR_CHECK(in.good(), "cannot read " << path);
  std::ostringstream ss;
  ss << in.rdbuf();
  return ss.str();
}

// Finds the Split pretokenizer's pattern in a pre_tokenizer entry (a Split,
// or a Sequence holding one); null when there is none.
const json::Value* find_split_pattern(const json::Value& p) {
  if (!p.is_object()) return nullptr;
  const json::Value* type = p.find("type");
  if (type != nullptr && type->is_string() && type->as_string() == "Split") {
    const json::Value* pattern = p.find("pattern");
    if (pattern != nullptr && pattern->is_object()) {
      const json::Value* rx = pattern->find("Regex");
      if (rx == nullptr) rx = pattern->find("String");
      return rx;
    }
    return nullptr;
  }
  const json::Value* list = p.find("pretokenizers");
  if (list != nullptr && list->is_array()) {
    for (const json::Value& item : list->items()) {
      if (const json::Value* rx = find_split_pattern(item)) return rx;
    }
  }
  return nullptr;
}

}  // namespace

std::vector<std::string> Tokenizer::split_pretokens(const std::string& text) {
  std::vector<std::string> out;
  const Chars t(text);
  size_t i = 0;
  while (i < t.size()) {
    const size_t len = match_at(t, i);
    out.push_back(text.substr(t.at[i], t.at[i + len] - t.at[i]));
    i += len;
  }
  return out;
}

std::string Tokenizer::byte_level_encode(const std::string& raw) {
  std::string out;
  out.reserve(raw.size() * 2);
  for (char c : raw) append_utf8(&out, alphabet().to_cp[static_cast<unsigned char>(c)]);
  return out;
}

std::string Tokenizer::byte_level_decode(const std::string& encoded) {
  std::string out;
  size_t i = 0;
  while (i < encoded.size()) {
    size_t len = 1;
    const uint32_t cp = next_code_point(encoded, i, &len);
    const auto hit = alphabet().to_byte.find(cp);
    if (hit != alphabet().to_byte.end()) {
      out.push_back(static_cast<char>(hit->second));
    } else {
      out.append(encoded, i, len);  // not a byte-level character: kept as written
    }
    i += len;
  }
  return out;
}

Tokenizer Tokenizer::from_model_dir(const std::string& model_dir) {
  return from_file(model_dir + "/tokenizer.json");
}

Tokenizer Tokenizer::from_file(const std::string& path) { return from_json_string(read_file(path)); }

Tokenizer Tokenizer::from_json_string(const std::string& text) {
  Tokenizer t;
  t.load(text);
  return t;
}

void Tokenizer::load(const std::string& text) {
  json::Value doc;
  std::string err;
  LCR_CHECK(json::parse(text, &doc, &err), "tokenizer.json is not valid JSON: " << err);
  const json::Value* model = doc.find("model");
  const std::string type =
      model != nullptr && model->find("type") != nullptr ? model->at("type").as_string() : std::string("none");
  LCR_CHECK(type == "BPE", "tokenizer.json model is " << type << "; this runtime only implements byte-level BPE");
  const json::Value* pre = doc.find("pre_tokenizer");
  const json::Value* pattern = pre != nullptr ? find_split_pattern(*pre) : nullptr;
  LCR_CHECK(pattern != nullptr,
            "tokenizer.json has no Split pretokenizer; this runtime implements the Llama 3 split pattern only");
  LCR_CHECK(pattern->is_string() && pattern->as_string() == kLlama3Pattern,
            "tokenizer.json uses a pretokenizer pattern this runtime does not implement: "
                << (pattern->is_string() ? pattern->as_string() : std::string("(not a string)")));
  if (const json::Value* im = model->find("ignore_merges")) ignore_merges_ = im->is_bool() && im->as_bool();

  auto place = [&](int id, const std::string& piece, uint8_t kind) {
    LCR_CHECK(id >= 0, "negative token id " << id << " in tokenizer.json");
    if (static_cast<size_t>(id) >= pieces_.size()) {
      pieces_.resize(static_cast<size_t>(id) + 1);
      kind_.resize(static_cast<size_t>(id) + 1, 0);
    }
    pieces_[static_cast<size_t>(id)] = piece;
    kind_[static_cast<size_t>(id)] = kind;
  };
  for (const auto& entry : model->at("vocab").members()) {
    const int id = entry.second.as_int();
    place(id, entry.first, 1);
    piece_id_[entry.first] = id;
  }
  const json::Value* merges = model->find("merges");
  if (merges != nullptr) {
    int rank = 0;
    for (const json::Value& m : merges->items()) {
      std::string left, right;
      if (m.is_string()) {
        const std::string& s = m.as_string();
        const size_t sp = s.find(' ');
        LCR_CHECK(sp != std::string::npos, "merge \"" << s << "\" has no separating space");
        left = s.substr(0, sp);
        right = s.substr(sp + 1);
      } else {
        LCR_CHECK(m.is_array() && m.size() == 2, "a merge is neither \"a b\" nor [\"a\", \"b\"]");
        left = m.items()[0].as_string();
        right = m.items()[1].as_string();
      }
      const auto l = piece_id_.find(left), r = piece_id_.find(right), res = piece_id_.find(left + right);
      if (l != piece_id_.end() && r != piece_id_.end() && res != piece_id_.end()) {
        merges_.emplace(pair_key(l->second, r->second), Merge{rank, res->second});
      }
      ++rank;
    }
  }
  if (const json::Value* added = doc.find("added_tokens")) {
    for (const json::Value& a : added->items()) {
      const int id = a.at("id").as_int();
      const std::string& content = a.at("content").as_string();
      const json::Value* sp = a.find("special");
      const bool special = sp != nullptr && sp->is_bool() && sp->as_bool();
      place(id, content, special ? 3 : 2);
      if (content.empty()) continue;
      added_.push_back(Added{content, id, special});
      added_first_byte_[static_cast<unsigned char>(content[0])] = true;
      if (content == "<|begin_of_text|>") bos_id_ = id;
    }
  }
  std::stable_sort(added_.begin(), added_.end(),
                   [](const Added& a, const Added& b) { return a.content.size() > b.content.size(); });
}

int Tokenizer::token_to_id(const std::string& token) const {
  const auto hit = piece_id_.find(token);
  if (hit != piece_id_.end()) return hit->second;
  for (const Added& a : added_) {
    if (a.content == token) return a.id;
  }
  return -1;
}

const std::string& Tokenizer::id_to_token(int id) const {
  LCR_CHECK(id >= 0 && id < vocab_size(), "token id " << id << " is outside the vocabulary of " << vocab_size());
  return pieces_[static_cast<size_t>(id)];
}

bool Tokenizer::is_special(int id) const {
  return id >= 0 && id < vocab_size() && kind_[static_cast<size_t>(id)] == 3;
}

void Tokenizer::bpe(const std::string& pretoken, std::vector<int>* out) const {
  const std::string piece = byte_level_encode(pretoken);
  if (ignore_merges_) {
    const auto whole = piece_id_.find(piece);
    if (whole != piece_id_.end()) {
      out->push_back(whole->second);
      return;
    }
  }
  // One symbol per byte-level character, linked both ways.
  std::vector<int> id, prev, next;
  size_t i = 0;
  while (i < piece.size()) {
    size_t len = 1;
    next_code_point(piece, i, &len);
    const auto hit = piece_id_.find(piece.substr(i, len));
    LCR_CHECK(hit != piece_id_.end(), "byte-level character \"" << piece.substr(i, len)
                                                                 << "\" is missing from the vocabulary");
    id.push_back(hit->second);
    i += len;
  }
  const int n = static_cast<int>(id.size());
  if (n == 0) return;
  for (int k = 0; k < n; ++k) {
    prev.push_back(k - 1);
    next.push_back(k + 1 < n ? k + 1 : -1);
  }
  // Candidate merges, lowest rank first, then leftmost. An entry is stale when
  // either symbol has changed since it was pushed.
  struct Cand {
    int rank, pos, left, right;
    bool operator<(const Cand& o) const { return rank != o.rank ? rank > o.rank : pos > o.pos; }
  };
  std::priority_queue<Cand> heap;
  auto consider = [&](int a) {
    if (a < 0 || next[static_cast<size_t>(a)] < 0) return;
    const int b = next[static_cast<size_t>(a)];
    const auto m = merges_.find(pair_key(id[static_cast<size_t>(a)], id[static_cast<size_t>(b)]));
    if (m != merges_.end()) heap.push(Cand{m->second.rank, a, id[static_cast<size_t>(a)], id[static_cast<size_t>(b)]});
  };
  for (int k = 0; k + 1 < n; ++k) consider(k);
  std::vector<char> dead(static_cast<size_t>(n), 0);
  while (!heap.empty()) {
    const Cand c = heap.top();
    heap.pop();
    const size_t a = static_cast<size_t>(c.pos);
    if (dead[a] || id[a] != c.left) continue;
    const int b = next[a];
    if (b < 0 || id[static_cast<size_t>(b)] != c.right) continue;
    id[a] = merges_.at(pair_key(c.left, c.right)).result;
    dead[static_cast<size_t>(b)] = 1;
    next[a] = next[static_cast<size_t>(b)];
    if (next[a] >= 0) prev[static_cast<size_t>(next[a])] = c.pos;
    consider(prev[a]);
    consider(c.pos);
  }
  for (int k = 0; k >= 0; k = next[static_cast<size_t>(k)]) out->push_back(id[static_cast<size_t>(k)]);
}

void Tokenizer::encode_span(const std::string& text, size_t begin, size_t end, std::vector<int>* out) const {
  if (end <= begin) return;
  for (const std::string& pre : split_pretokens(text.substr(begin, end - begin))) bpe(pre, out);
}

std::vector<int> Tokenizer::encode(const std::string& text, bool add_bos, bool parse_special) const {
  std::vector<int> out;
  if (add_bos) {
    LCR_CHECK(bos_id_ >= 0, "this tokenizer has no <|begin_of_text|> token to prepend");
    out.push_back(bos_id_);
  }
  size_t span = 0;
  size_t i = 0;
  while (parse_special && i < text.size()) {
    const Added* hit = nullptr;
    if (added_first_byte_[static_cast<unsigned char>(text[i])]) {
      for (const Added& a : added_) {  // longest first
        if (text.compare(i, a.content.size(), a.content) == 0) {
          hit = &a;
          break;
        }
      }
    }
    if (hit == nullptr) {
      ++i;
      continue;
    }
    encode_span(text, span, i, &out);
    out.push_back(hit->id);
    i += hit->content.size();
    span = i;
  }
  encode_span(text, span, text.size(), &out);
  return out;
}

std::string Tokenizer::decode_one(int id, bool skip_special) const {
  LCR_CHECK(id >= 0 && id < vocab_size(), "token id " << id << " is outside the vocabulary of " << vocab_size());
  const uint8_t kind = kind_[static_cast<size_t>(id)];
  if (kind == 3 && skip_special) return std::string();
  if (kind == 2 || kind == 3) return pieces_[static_cast<size_t>(id)];
  return byte_level_decode(pieces_[static_cast<size_t>(id)]);
}

std::string Tokenizer::decode(const std::vector<int>& ids, bool skip_special) const {
  std::string out;
  for (int id : ids) out += decode_one(id, skip_special);
  return out;
}

}  // namespace lcr
