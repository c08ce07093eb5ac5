// Byte-fallback BPE tokenizer read from a Hugging Face tokenizer.json, the
// C++ counterpart of fiber/ai's tokenizer package (tokenizer/tokenizer.go,
// tokenizer/trie.go). It accepts exactly the pieces the Gemma files use and
// refuses anything else at load time, as the reference does:
//   model BPE (byte_fallback optional), merges as "a b" strings or [a, b]
//   pairs; normalizer Replace (or none); pre_tokenizer Split on " ",
//   Metaspace or none; added tokens with normalized == false; post-processor
//   TemplateProcessing whose single template is [BOS] A [EOS].
// Encoding: added tokens are matched literally in the raw text, longest
// first; the text between them is normalized and run through BPE, which
// repeatedly merges the adjacent pair of lowest merge rank (the leftmost on
// ties); characters outside the vocab become their UTF-8 byte tokens
// <0xNN> (byte_fallback) or <unk>. Invalid UTF-8 bytes read as U+FFFD.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace fiber::json {
class Value;
}

namespace fiber::tokenizer {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

class Tokenizer {
 public:
  // Reads a tokenizer.json file (tokenizer.go:46 Load).
  static Tokenizer Load(const std::string& path);
  // Parses tokenizer.json text (tokenizer.go:80 parse).
  static Tokenizer Parse(const std::string& json_text);

  // Token ids with the file's BOS/EOS template (tokenizer.go:296).
  std::vector<int> Encode(const std::string& text) const;
  // Token ids without the template (tokenizer.go:312).
  std::vector<int> EncodeRaw(const std::string& text) const;
  // Text of ids: byte tokens become their bytes, the metaspace becomes a
  // space, added tokens render literally (tokenizer.go:468).
  std::string Decode(const std::vector<int>& ids) const;

  int BOS() const { return bos_; }  // -1 when the template adds none
  int EOS() const { return eos_; }
  int VocabSize() const { return (int)pieces_.size(); }  // highest id + 1
  std::string Piece(int id) const;
  bool ID(const std::string& piece, int* id) const;
  // The normalizer's replacement (the metaspace for Gemma files).
  const std::string& NormalizedSpace() const { return norm_to_; }

 private:
  struct Merge {
    int32_t rank, merged;
  };
  struct TrieNode {
    std::vector<std::pair<unsigned char, int32_t>> kids;  // byte -> node, sorted
    int32_t id = -1;                                       // added-token id ending here
  };

  std::unordered_map<std::string, int32_t> vocab_;
  std::vector<std::string> pieces_;
  std::unordered_map<uint64_t, Merge> merges_;  // (left id, right id) -> merge
  std::vector<TrieNode> trie_;
  std::unordered_map<int32_t, std::string> added_;
  std::string norm_from_, norm_to_;
  bool byte_fallback_ = false;
  int32_t byte_tok_[256] = {};
  std::unordered_map<int32_t, uint8_t> byte_of_;
  int32_t unk_ = -1;
  int32_t bos_ = -1, eos_ = -1;
  bool add_bos_ = false, add_eos_ = false;

  static Tokenizer parse_doc(const json::Value& doc);
  void trie_insert(const std::string& s, int32_t id);
  // Longest added token at s[i..]: its id and byte length, or length 0.
  std::pair<int32_t, size_t> trie_longest(const std::string& s, size_t i) const;
  void encode(const std::string& text, std::vector<int32_t>& out) const;
  void bpe(const std::string& chunk, std::vector<int32_t>& out) const;
};

}  // namespace fiber::tokenizer
