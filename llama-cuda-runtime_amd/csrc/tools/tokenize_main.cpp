// lcr-tokenize: the tokenizer on a stream of texts, for diffing against
// another implementation (the reference's tools/tokenize_main.cpp interface):
//
//   lcr-tokenize <tokenizer.json> [--no-special] [--add-bos] < corpus.jsonl
//
// Every non-empty input line is a JSON string; the output line is its token
// ids separated by spaces, or ROUNDTRIP_FAILED when decoding them does not
// give the text back.
#include <cstdio>
#include <iostream>
#include <string>
#include <vector>

#include "../json.h"
#include "../tokenizer.h"

int main(int argc, char** argv) {
  std::string path;
  bool parse_special = true, add_bos = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--no-special") parse_special = false;
    else if (a == "--add-bos") add_bos = true;
    else if (path.empty()) path = a;
    else {
      std::fprintf(stderr, "unexpected argument: %s\n", a.c_str());
      return 2;
    }
  }
  if (path.empty()) {
    std::fprintf(stderr, "usage: lcr-tokenize <tokenizer.json> [--no-special] [--add-bos] < corpus.jsonl\n");
    return 2;
  }
  try {
    const lcr::Tokenizer tok = lcr::Tokenizer::from_file(path);
    std::ios::sync_with_stdio(false);
    std::string line;
    while (std::getline(std::cin, line)) {
      if (line.empty()) continue;
      lcr::json::Value v;
      std::string err;
      if (!lcr::json::parse(line, &v, &err) || !v.is_string()) {
        std::fprintf(stderr, "input line is not a JSON string: %s\n", line.c_str());
        return 2;
      }
      const std::string& text = v.as_string();
      // The begin-of-text token decodes to its own text, which the input
      // did not hold.
      const std::vector<int> ids = tok.encode(text, add_bos, parse_special);
      const std::vector<int> body(ids.begin() + (add_bos ? 1 : 0), ids.end());
      if (tok.decode(body) != text) {
        std::cout << "ROUNDTRIP_FAILED\n";
        continue;
      }
      for (size_t i = 0; i < ids.size(); ++i) std::cout << (i ? " " : "") << ids[i];
      std::cout << '\n';
    }
    std::cout.flush();
  } catch (const std::exception& e) {
    std::fprintf(stderr, "%s\n", e.what());
    return 1;
  }
  return 0;
}
