// fiber::tokenizer::Tokenizer (ai_amd/host/tokenizer.hpp) on the CPU:
// the reference's own synthetic tests (tokenizer/synthetic_test.go),
// parity with Hugging Face `tokenizers` on the committed golden cases
// (tests/golden/tokenizer_golden.json, made by make_tokenizer_golden.py),
// the round trip (tokenizer/tokenizer_test.go:101-121) and edge cases.
// Run from the repository root by tests/test_cpp_host.py.
#include <cstdio>
#include <fstream>
#include <sstream>

#include "json.hpp"
#include "testing.hpp"
#include "tokenizer.hpp"

using fiber::tokenizer::Tokenizer;
namespace json = fiber::json;

static std::string ids_str(const std::vector<int>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); i++) s += (i ? " " : "") + std::to_string(v[i]);
  return s + "]";
}

// The reference's buildTokenizer (synthetic_test.go:13-60) as JSON text.
static std::string synthetic_json(const std::string& model_override = "", const std::string& extra = "") {
  std::string vocab = R"("<pad>":0,"<eos>":1,"<bos>":2,"<unk>":3,"▁":4,"a":5,"b":6,"c":7,"ab":8,"abc":9,"▁a":10)";
  for (int b = 0; b < 256; b++) {
    char k[32];
    std::snprintf(k, sizeof k, ",\"<0x%02X>\":%d", b, 11 + b);
    vocab += k;
  }
  std::string model = model_override.empty()
                          ? R"({"type":"BPE","unk_token":"<unk>","byte_fallback":true,"ignore_merges":false,"vocab":{)" +
                                vocab + R"(},"merges":[["a","b"],["ab","c"],["▁","a"]]})"
                          : model_override;
  return R"({"added_tokens":[{"id":2,"content":"<bos>","special":true,"normalized":false},)"
         R"({"id":1,"content":"<eos>","special":true,"normalized":false},)"
         R"({"id":0,"content":"<pad>","special":true,"normalized":false}],)"
         R"("normalizer":{"type":"Replace","pattern":{"String":" "},"content":"▁"},)"
         R"("pre_tokenizer":{"type":"Split","pattern":{"String":" "},"behavior":"MergedWithPrevious"},)"
         R"("post_processor":{"type":"TemplateProcessing","single":[{"SpecialToken":{"id":"<bos>","type_id":0}},)"
         R"({"Sequence":{"id":"A","type_id":0}},{"SpecialToken":{"id":"<eos>","type_id":0}}]},)" +
         extra + R"("model":)" + model + "}";
}

// tokenizer/synthetic_test.go:62-101
TEST(TestSyntheticBPE) {
  Tokenizer tok = Tokenizer::Parse(synthetic_json());
  const struct {
    const char* in;
    std::vector<int> raw;
  } cases[] = {
      {"abc", {9}}, {"ab", {8}}, {"ba", {6, 5}}, {"a", {5}}, {" a", {10}}, {"", {}},
      {"Z", {11 + 'Z'}}, {"\xc3\xa9", {11 + 0xC3, 11 + 0xA9}},
  };
  for (const auto& c : cases) {
    const auto got = tok.EncodeRaw(c.in);
    if (got != c.raw) FATAL("EncodeRaw(%s) = %s, want %s", c.in, ids_str(got).c_str(), ids_str(c.raw).c_str());
  }
  if (tok.Encode("abc") != std::vector<int>{2, 9, 1}) FATAL("Encode(abc) = %s", ids_str(tok.Encode("abc")).c_str());
  if (tok.EncodeRaw("a<bos>b") != std::vector<int>{5, 2, 6}) FATAL("added split = %s", ids_str(tok.EncodeRaw("a<bos>b")).c_str());
  if (tok.Decode(tok.EncodeRaw("abc \xc3\xa9")) != "abc \xc3\xa9") FATAL("decode = %s", tok.Decode(tok.EncodeRaw("abc \xc3\xa9")).c_str());
  if (tok.BOS() != 2 || tok.EOS() != 1) FATAL("bos/eos %d/%d", tok.BOS(), tok.EOS());
}

// tokenizer/synthetic_test.go:103-129
TEST(TestLoadErrors) {
  const struct {
    const char* name;
    std::string doc;
    const char* want;
  } cases[] = {
      {"model type", R"({"model":{"type":"WordPiece","vocab":{"a":0}}})", "model type"},
      {"normalizer",
       R"({"model":{"type":"BPE","byte_fallback":false,"vocab":{"a":0},"merges":[]},"normalizer":{"type":"NFKC"}})",
       "normalizer"},
      {"pre_tokenizer",
       R"({"model":{"type":"BPE","byte_fallback":false,"vocab":{"a":0},"merges":[]},"pre_tokenizer":{"type":"ByteLevel"}})",
       "pre_tokenizer"},
      {"missing byte token", R"({"model":{"type":"BPE","byte_fallback":true,"vocab":{"a":0},"merges":[]}})",
       "byte_fallback"},
      {"empty vocab", R"({"model":{"type":"BPE","vocab":{},"merges":[]}})", "empty vocab"},
  };
  for (const auto& c : cases) {
    try {
      Tokenizer::Parse(c.doc);
      FATAL("%s: no error", c.name);
    } catch (const fiber::tokenizer::Error& e) {
      if (std::string(e.what()).find(c.want) == std::string::npos) FATAL("%s: err %s, want %s", c.name, e.what(), c.want);
    }
  }
  try {
    Tokenizer::Parse("{\"model\": ");
    FATAL("truncated JSON: no error");
  } catch (const fiber::tokenizer::Error&) {
  }
}

static json::Value golden() {
  return json::parse_file("tests/golden/tokenizer_golden.json");
}

TEST(TestGoldenHuggingFaceParity) {
  const json::Value g = golden();
  std::vector<std::pair<std::string, Tokenizer>> toks;
  for (const auto& kv : g.at("files").members()) toks.emplace_back(kv.first, Tokenizer::Parse(kv.second.as_string()));
  int n = 0;
  for (const json::Value& c : g.at("cases").items()) {
    const std::string& name = c.at("tok").as_string();
    const Tokenizer* tok = nullptr;
    for (auto& t : toks)
      if (t.first == name) tok = &t.second;
    if (!tok) FATAL("no tokenizer %s", name.c_str());
    const std::string& s = c.at("s").as_string();
    std::vector<int> want, want_raw;
    for (const auto& v : c.at("ids").items()) want.push_back((int)v.as_int());
    for (const auto& v : c.at("raw").items()) want_raw.push_back((int)v.as_int());
    const auto got = tok->Encode(s), got_raw = tok->EncodeRaw(s);
    if (got != want) FATAL("%s Encode(\"%s\") = %s, want %s", name.c_str(), s.c_str(), ids_str(got).c_str(), ids_str(want).c_str());
    if (got_raw != want_raw)
      FATAL("%s EncodeRaw(\"%s\") = %s, want %s", name.c_str(), s.c_str(), ids_str(got_raw).c_str(), ids_str(want_raw).c_str());
    n++;
  }
  if (n < 100) FATAL("only %d golden cases", n);
  std::printf("    %d cases identical to Hugging Face tokenizers\n", n);
}

// tokenizer/tokenizer_test.go:101-121: raw text round-trips unless it holds
// a literal metaspace.
TEST(TestRoundTrip) {
  const json::Value g = golden();
  Tokenizer tok = Tokenizer::Parse(g.at("files").at("learned").as_string());
  int n = 0;
  for (const json::Value& c : g.at("cases").items()) {
    if (c.at("tok").as_string() != "learned") continue;
    const std::string& s = c.at("s").as_string();
    if (s.find(tok.NormalizedSpace()) != std::string::npos) continue;
    const std::string back = tok.Decode(tok.EncodeRaw(s));
    if (back != s) FATAL("round trip \"%s\" -> \"%s\"", s.c_str(), back.c_str());
    n++;
  }
  if (n < 50) FATAL("only %d round trips", n);
}

TEST(TestEdgeCases) {
  // a merge naming a piece outside the vocab cannot fire and is skipped
  std::string vocab = R"("a":0,"b":1,"ab":2)";
  Tokenizer t = Tokenizer::Parse(R"({"model":{"type":"BPE","vocab":{)" + vocab +
                                 R"(},"merges":["zz qq","a b"]}})");
  if (t.EncodeRaw("ab") != std::vector<int>{2}) FATAL("merge after a skipped one: %s", ids_str(t.EncodeRaw("ab")).c_str());
  if (t.BOS() != -1 || t.EOS() != -1) FATAL("no template: bos/eos %d/%d", t.BOS(), t.EOS());
  if (t.Encode("ab") != std::vector<int>{2}) FATAL("no template adds nothing");
  // invalid UTF-8 reads as U+FFFD, whose bytes EF BF BD fall back
  Tokenizer s = Tokenizer::Parse(synthetic_json());
  const std::vector<int> want = {11 + 0xEF, 11 + 0xBF, 11 + 0xBD, 5};
  if (s.EncodeRaw("\xff" "a") != want) FATAL("invalid byte: %s", ids_str(s.EncodeRaw("\xff" "a")).c_str());
  // an added token that stops inside a multi-byte character is not a match
  Tokenizer u = Tokenizer::Parse(synthetic_json("", R"("x_unused":0,)"));
  if (u.VocabSize() != 267) FATAL("vocab size %d", u.VocabSize());
  // merges in "a b" string form equal the pair form
  std::string v2;
  for (int b = 0; b < 256; b++) {
    char k[32];
    std::snprintf(k, sizeof k, ",\"<0x%02X>\":%d", b, 11 + b);
    v2 += k;
  }
  Tokenizer w = Tokenizer::Parse(synthetic_json(
      R"({"type":"BPE","byte_fallback":true,"vocab":{"<pad>":0,"<eos>":1,"<bos>":2,"<unk>":3,"▁":4,"a":5,"b":6,"c":7,"ab":8,"abc":9,"▁a":10)" +
      v2 + R"(},"merges":["a b","ab c","▁ a"]})"));
  if (w.EncodeRaw("abc ab") != std::vector<int>{9, 4, 8}) FATAL("string merges: %s", ids_str(w.EncodeRaw("abc ab")).c_str());
}

int main(int argc, char** argv) { return ctest::run_all(argc, argv); }
