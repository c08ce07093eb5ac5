// Loads a model directory with fiber::gemma::Model::Load and writes the
// embeddings of the texts in a JSON array file as raw fp32 rows:
//   embed_dir <model_dir> <texts.json> <out.f32> [prompt_name|-] [dim]
// Prints the embedding width and row count, or "error: ..." (exit 1).
// Driven by tests/test_gpu_load_embed.py.
#include <cstdio>
#include <cstdlib>

#include "fiber.hpp"
#include "json.hpp"

int main(int argc, char** argv) {
  if (argc < 4) {
    std::fprintf(stderr, "usage: embed_dir <model_dir> <texts.json> <out.f32> [prompt|-] [dim]\n");
    return 2;
  }
  try {
    auto model = fiber::gemma::Model::Load(argv[1]);
    std::vector<std::string> texts;
    const fiber::json::Value doc = fiber::json::parse_file(argv[2]);  // keep it alive while iterating
    for (const auto& v : doc.items()) texts.push_back(v.as_string());
    fiber::gemma::EmbedOpts o;
    if (argc > 4 && std::string(argv[4]) != "-") o.Prompt = argv[4];
    if (argc > 5) o.Dim = std::atoi(argv[5]);
    const auto emb = model->Embed(texts, o);
    FILE* f = std::fopen(argv[3], "wb");
    if (!f) throw std::runtime_error(std::string("cannot write ") + argv[3]);
    for (const auto& row : emb) std::fwrite(row.data(), 4, row.size(), f);
    std::fclose(f);
    std::printf("dim %zu rows %zu\n", emb.empty() ? 0 : emb[0].size(), emb.size());
  } catch (const std::exception& e) {
    std::printf("error: %s\n", e.what());
    return 1;
  }
  return 0;
}
