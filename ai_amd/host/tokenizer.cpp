#include "tokenizer.hpp"

#include <algorithm>
#include <cstdio>
#include <queue>

#include "json.hpp"

namespace fiber::tokenizer {

namespace {

uint64_t pair_key(int32_t l, int32_t r) { return ((uint64_t)(uint32_t)l << 32) | (uint32_t)r; }

// Decodes one code point at s[i] with the strict UTF-8 rules (no overlong
// forms, no surrogates, at most U+10FFFF); an invalid sequence reads as
// U+FFFD of length 1.
uint32_t decode_rune(const std::string& s, size_t i, size_t* len) {
  const unsigned char c0 = (unsigned char)s[i];
  auto cont = [&](size_t k) { return i + k < s.size() && ((unsigned char)s[i + k] & 0xC0) == 0x80; };
  *len = 1;
  if (c0 < 0x80) return c0;
  if (c0 >= 0xC2 && c0 <= 0xDF && cont(1)) {
    *len = 2;
    return ((c0 & 0x1Fu) << 6) | ((unsigned char)s[i + 1] & 0x3Fu);
  }
  if (c0 >= 0xE0 && c0 <= 0xEF && cont(1) && cont(2)) {
    const unsigned char c1 = (unsigned char)s[i + 1];
    if ((c0 == 0xE0 && c1 < 0xA0) || (c0 == 0xED && c1 >= 0xA0)) return 0xFFFD;
    *len = 3;
    return ((c0 & 0x0Fu) << 12) | ((c1 & 0x3Fu) << 6) | ((unsigned char)s[i + 2] & 0x3Fu);
  }
  if (c0 >= 0xF0 && c0 <= 0xF4 && cont(1) && cont(2) && cont(3)) {
    const unsigned char c1 = (unsigned char)s[i + 1];
    if ((c0 == 0xF0 && c1 < 0x90) || (c0 == 0xF4 && c1 >= 0x90)) return 0xFFFD;
    *len = 4;
    return ((c0 & 0x07u) << 18) | ((c1 & 0x3Fu) << 12) | (((unsigned char)s[i + 2] & 0x3Fu) << 6) |
           ((unsigned char)s[i + 3] & 0x3Fu);
  }
  return 0xFFFD;
}

std::string encode_rune(uint32_t cp) {
  std::string o;
  if (cp < 0x80) {
    o += (char)cp;
  } else if (cp < 0x800) {
    o += (char)(0xC0 | (cp >> 6));
    o += (char)(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    o += (char)(0xE0 | (cp >> 12));
    o += (char)(0x80 | ((cp >> 6) & 0x3F));
    o += (char)(0x80 | (cp & 0x3F));
  } else {
    o += (char)(0xF0 | (cp >> 18));
    o += (char)(0x80 | ((cp >> 12) & 0x3F));
    o += (char)(0x80 | ((cp >> 6) & 0x3F));
    o += (char)(0x80 | (cp & 0x3F));
  }
  return o;
}

std::string replace_all(const std::string& s, const std::string& from, const std::string& to) {
  if (from.empty()) return s;
  std::string out;
  size_t i = 0;
  for (;;) {
    const size_t j = s.find(from, i);
    if (j == std::string::npos) break;
    out.append(s, i, j - i);
    out += to;
    i = j + from.size();
  }
  out.append(s, i, std::string::npos);
  return out;
}

}  // namespace

Tokenizer Tokenizer::Load(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) throw Error("tokenizer: cannot open " + path);
  std::string text;
  char buf[1 << 16];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
  std::fclose(f);
  return Parse(text);
}

Tokenizer Tokenizer::Parse(const std::string& json_text) {
  try {
    return parse_doc(json::parse(json_text));
  } catch (const json::Error& e) {  // malformed JSON or a value of the wrong type
    throw Error(std::string("tokenizer: ") + e.what());
  }
}

Tokenizer Tokenizer::parse_doc(const json::Value& doc) {
  Tokenizer t;
  const json::Value& model = doc.at("model");
  const std::string type = model.get_string("type");
  if (type != "BPE") throw Error("tokenizer: model type \"" + type + "\" not supported (want BPE)");
  const json::Value* vocab = model.find("vocab");
  if (!vocab || !vocab->is_object() || vocab->members().empty()) throw Error("tokenizer: empty vocab");
  int32_t max_id = -1;
  for (const auto& kv : vocab->members()) {
    const int32_t id = (int32_t)kv.second.as_int();
    if (id < 0) throw Error("tokenizer: negative id for \"" + kv.first + "\"");
    t.vocab_.emplace(kv.first, id);
    max_id = std::max(max_id, id);
  }
  t.pieces_.assign((size_t)max_id + 1, std::string());
  for (const auto& kv : t.vocab_) t.pieces_[kv.second] = kv.first;
  t.byte_fallback_ = model.get_bool("byte_fallback");
  {
    auto it = t.vocab_.find("<unk>");
    if (it != t.vocab_.end()) t.unk_ = it->second;
  }

  // normalizer: Replace or none
  if (const json::Value* n = doc.find("normalizer"); n && !n->is_null()) {
    const std::string nt = n->get_string("type");
    if (nt != "Replace") throw Error("tokenizer: normalizer \"" + nt + "\" not supported (want Replace)");
    t.norm_from_ = n->at("pattern").get_string("String");
    t.norm_to_ = n->get_string("content");
  }
  // pre_tokenizer: a Split on a literal space never fires after the
  // space -> metaspace normalizer, so BPE runs over whole chunks
  if (const json::Value* p = doc.find("pre_tokenizer"); p && !p->is_null()) {
    const std::string pt = p->get_string("type");
    if (pt == "Split") {
      const json::Value* pat = p->find("pattern");
      const std::string ps = pat ? pat->get_string("String") : "";
      if (ps != " ") throw Error("tokenizer: pre_tokenizer Split on \"" + ps + "\" not supported");
    } else if (!(pt == "Metaspace" || pt.empty())) {
      throw Error("tokenizer: pre_tokenizer \"" + pt + "\" not supported");
    }
  }
  // merges: ["a b", ...] or [["a", "b"], ...]; a merge naming a piece outside
  // the vocab cannot fire and is skipped; the first rank of a pair wins
  const json::Value* merges = model.find("merges");
  if (!merges || !merges->is_array()) throw Error("tokenizer: no merges");
  int32_t rank = 0;
  for (const json::Value& m : merges->items()) {
    std::string l, r;
    if (m.is_array()) {
      if (m.items().size() != 2) throw Error("tokenizer: bad merge pair");
      l = m.items()[0].as_string();
      r = m.items()[1].as_string();
    } else {
      const std::string& line = m.as_string();
      const size_t sp = line.find(' ');
      if (sp == std::string::npos) throw Error("tokenizer: bad merge line \"" + line + "\"");
      l = line.substr(0, sp);
      r = line.substr(sp + 1);
    }
    const int32_t this_rank = rank++;
    auto il = t.vocab_.find(l), ir = t.vocab_.find(r), im = t.vocab_.find(l + r);
    if (il == t.vocab_.end() || ir == t.vocab_.end() || im == t.vocab_.end()) continue;
    t.merges_.emplace(pair_key(il->second, ir->second), Merge{this_rank, im->second});
  }
  if (t.byte_fallback_) {
    for (int b = 0; b < 256; b++) {
      char key[8];
      std::snprintf(key, sizeof key, "<0x%02X>", b);
      auto it = t.vocab_.find(key);
      if (it == t.vocab_.end())
        throw Error(std::string("tokenizer: byte_fallback set but ") + key + " is missing from the vocab");
      t.byte_tok_[b] = it->second;
      t.byte_of_[it->second] = (uint8_t)b;
    }
  }
  t.trie_.emplace_back();  // root
  if (const json::Value* added = doc.find("added_tokens"); added && added->is_array()) {
    for (const json::Value& a : added->items()) {
      const std::string content = a.get_string("content");
      if (a.get_bool("normalized"))
        throw Error("tokenizer: added token \"" + content + "\" is normalized; only raw added tokens are supported");
      const int32_t id = (int32_t)a.get_int("id", -1);
      t.trie_insert(content, id);
      t.added_[id] = content;
    }
  }
  // post-processor: the special token before the sequence is BOS, after EOS
  if (const json::Value* pp = doc.find("post_processor"); pp && !pp->is_null()) {
    const std::string ptype = pp->get_string("type");
    if (!ptype.empty() && ptype != "TemplateProcessing")
      throw Error("tokenizer: post-processor \"" + ptype + "\" not supported");
    if (const json::Value* single = pp->find("single"); single && single->is_array()) {
      bool seen_seq = false;
      for (const json::Value& e : single->items()) {
        if (e.find("Sequence")) {
          seen_seq = true;
          continue;
        }
        const json::Value* st = e.find("SpecialToken");
        if (!st) continue;
        const std::string name = st->get_string("id");
        auto it = t.vocab_.find(name);
        if (it == t.vocab_.end()) throw Error("tokenizer: template special token \"" + name + "\" not in vocab");
        if (!seen_seq) {
          t.bos_ = it->second;
          t.add_bos_ = true;
        } else {
          t.eos_ = it->second;
          t.add_eos_ = true;
        }
      }
    }
  }
  return t;
}

void Tokenizer::trie_insert(const std::string& s, int32_t id) {
  if (s.empty()) return;
  int32_t node = 0;
  for (unsigned char c : s) {
    auto& kids = trie_[node].kids;
    auto it = std::lower_bound(kids.begin(), kids.end(), std::make_pair(c, (int32_t)-1),
                               [](const auto& a, const auto& b) { return a.first < b.first; });
    if (it != kids.end() && it->first == c) {
      node = it->second;
    } else {
      const int32_t fresh = (int32_t)trie_.size();
      kids.insert(it, {c, fresh});
      trie_.emplace_back();
      node = fresh;
    }
  }
  trie_[node].id = id;
}

std::pair<int32_t, size_t> Tokenizer::trie_longest(const std::string& s, size_t i) const {
  int32_t node = 0, best = -1;
  size_t best_len = 0;
  for (size_t k = i; k < s.size(); k++) {
    const auto& kids = trie_[node].kids;
    const unsigned char c = (unsigned char)s[k];
    auto it = std::lower_bound(kids.begin(), kids.end(), std::make_pair(c, (int32_t)-1),
                               [](const auto& a, const auto& b) { return a.first < b.first; });
    if (it == kids.end() || it->first != c) break;
    node = it->second;
    if (trie_[node].id >= 0) {
      best = trie_[node].id;
      best_len = k - i + 1;
    }
  }
  // a match must end on a character boundary (tokenizer/trie.go:57-70)
  if (best_len > 0 && i + best_len < s.size() && ((unsigned char)s[i + best_len] & 0xC0) == 0x80) return {0, 0};
  return {best, best_len};
}

std::string Tokenizer::Piece(int id) const {
  if (id < 0 || id >= (int)pieces_.size()) return std::string();
  return pieces_[id];
}

bool Tokenizer::ID(const std::string& piece, int* id) const {
  auto it = vocab_.find(piece);
  if (it == vocab_.end()) return false;
  *id = it->second;
  return true;
}

void Tokenizer::bpe(const std::string& chunk, std::vector<int32_t>& out) const {
  if (chunk.empty()) return;
  // initial symbols: one per character, or its byte tokens, or <unk>
  std::vector<int32_t> id;
  id.reserve(chunk.size());
  for (size_t i = 0; i < chunk.size();) {
    size_t len;
    const uint32_t cp = decode_rune(chunk, i, &len);
    const std::string ch = encode_rune(cp);
    i += len;
    auto it = vocab_.find(ch);
    if (it != vocab_.end()) {
      id.push_back(it->second);
    } else if (byte_fallback_) {
      for (unsigned char b : ch) id.push_back(byte_tok_[b]);
    } else if (unk_ >= 0) {
      id.push_back(unk_);
    }
  }
  const int32_t n = (int32_t)id.size();
  if (n == 0) return;
  std::vector<int32_t> prev(n), next(n);
  std::vector<char> alive(n, 1);
  for (int32_t i = 0; i < n; i++) {
    prev[i] = i - 1;
    next[i] = i + 1 < n ? i + 1 : -1;
  }
  // candidate pairs ordered by (rank, left position); stale entries are
  // skipped when popped
  struct Cand {
    int32_t rank, pos, l, r;
  };
  auto later = [](const Cand& a, const Cand& b) { return a.rank != b.rank ? a.rank > b.rank : a.pos > b.pos; };
  std::priority_queue<Cand, std::vector<Cand>, decltype(later)> heap(later);
  auto consider = [&](int32_t pos) {
    if (pos < 0) return;
    const int32_t nx = next[pos];
    if (nx < 0) return;
    auto it = merges_.find(pair_key(id[pos], id[nx]));
    if (it != merges_.end()) heap.push(Cand{it->second.rank, pos, id[pos], id[nx]});
  };
  for (int32_t i = 0; i < n; i++) consider(i);
  while (!heap.empty()) {
    const Cand c = heap.top();
    heap.pop();
    if (!alive[c.pos] || id[c.pos] != c.l) continue;
    const int32_t j = next[c.pos];
    if (j < 0 || !alive[j] || id[j] != c.r) continue;
    id[c.pos] = merges_.at(pair_key(c.l, c.r)).merged;
    alive[j] = 0;
    next[c.pos] = next[j];
    if (next[j] >= 0) prev[next[j]] = c.pos;
    consider(c.pos);
    consider(prev[c.pos]);
  }
  for (int32_t i = 0; i >= 0; i = next[i]) out.push_back(id[i]);
}

void Tokenizer::encode(const std::string& text, std::vector<int32_t>& out) const {
  std::string pending;
  auto flush = [&]() {
    if (pending.empty()) return;
    bpe(replace_all(pending, norm_from_, norm_to_), out);
    pending.clear();
  };
  for (size_t i = 0; i < text.size();) {
    const auto [aid, alen] = trie_longest(text, i);
    if (alen > 0) {
      flush();
      out.push_back(aid);
      i += alen;
      continue;
    }
    size_t len;
    decode_rune(text, i, &len);
    pending.append(text, i, len);
    i += len;
  }
  flush();
}

std::vector<int> Tokenizer::EncodeRaw(const std::string& text) const {
  std::vector<int32_t> ids;
  encode(text, ids);
  return std::vector<int>(ids.begin(), ids.end());
}

std::vector<int> Tokenizer::Encode(const std::string& text) const {
  std::vector<int32_t> ids;
  encode(text, ids);
  std::vector<int> out;
  out.reserve(ids.size() + 2);
  if (add_bos_) out.push_back(bos_);
  out.insert(out.end(), ids.begin(), ids.end());
  if (add_eos_) out.push_back(eos_);
  return out;
}

std::string Tokenizer::Decode(const std::vector<int>& ids) const {
  std::string out;
  for (int id : ids) {
    auto b = byte_of_.find(id);
    if (b != byte_of_.end()) {
      out += (char)b->second;
      continue;
    }
    out += norm_to_.empty() ? Piece(id) : replace_all(Piece(id), norm_to_, norm_from_);
  }
  return out;
}

}  // namespace fiber::tokenizer
