// Drives Transformer::load(const Model&, quant::Type) -- the reference's
// signature (include/llmi/model/transformer.hpp:58), implemented by
// host/integration/load_from_model.cpp -- on a model directory read by the
// reference's own Model::load (src/model/model.cpp), then runs one session on
// the GPU and writes what it produced, for tests/test_gpu_load_from_model.py
// to compare with the reference's logits:
//
//   load_from_model_check DIR TYPE OUT PROMPT_IDS STEP_IDS
//
// TYPE: f32 | q8_0 | q4_0; PROMPT_IDS / STEP_IDS: comma-separated token ids.
// OUT receives, as raw little-endian arrays: the prefill's logits at every
// prompt position (float32), the logits of each single-token step (float32),
// then the int32 ids of a 12-token greedy generation from the prompt 1, 2, 3.
// Exit status 0 on success; 2 with the reference's or the library's message
// on stderr otherwise.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "llmi/model/model.hpp"
#include "llmi/model/transformer.hpp"

namespace {

std::vector<llmi::TokenId> ids_of(const std::string& s) {
  std::vector<llmi::TokenId> out;
  std::size_t pos = 0;
  while (pos < s.size()) {
    const std::size_t end = s.find(',', pos);
    out.push_back(static_cast<llmi::TokenId>(std::stol(s.substr(pos, end - pos))));
    if (end == std::string::npos) break;
    pos = end + 1;
  }
  return out;
}

int die(const std::string& what) {
  std::fprintf(stderr, "%s\n", what.c_str());
  return 2;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 6) return die("usage: load_from_model_check DIR TYPE OUT PROMPT_IDS STEP_IDS");
  const std::string type = argv[2];
  const llmi::quant::Type qt = type == "q8_0"   ? llmi::quant::Type::Q8_0
                               : type == "q4_0" ? llmi::quant::Type::Q4_0
                                                : llmi::quant::Type::F32;
  auto model = llmi::Model::load(argv[1]);
  if (!model) return die("Model::load: " + model.error());
  auto tf = llmi::Transformer::load(*model, qt);
  if (!tf) return die("Transformer::load: " + tf.error());
  const auto prompt = ids_of(argv[4]);
  const auto steps = ids_of(argv[5]);
  auto cache = tf->new_cache(prompt.size() + steps.size());
  if (!cache) return die(cache.error());
  std::FILE* out = std::fopen(argv[3], "wb");
  if (out == nullptr) return die(std::string("cannot write ") + argv[3]);
  auto pre = tf->forward_cached(prompt, *cache, true);
  if (!pre) return die(pre.error());
  std::fwrite(pre->data(), sizeof(float), pre->size(), out);
  for (const llmi::TokenId s : steps) {
    auto step = tf->forward_cached({s}, *cache);
    if (!step) return die(step.error());
    std::fwrite(step->data(), sizeof(float), step->size(), out);
  }
  auto ids = tf->generate_greedy_cached({1, 2, 3}, 12, {});
  if (!ids) return die(ids.error());
  std::fwrite(ids->data(), sizeof(llmi::TokenId), ids->size(), out);
  std::fclose(out);
  return 0;
}
