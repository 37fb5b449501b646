// Drives the model-file parser (katago_amd/host/neuralnet/desc.cpp) under
// the host sanitizers. Every model named on the command line is parsed as
// given (.bin.gz / .txt.gz); then each is decompressed and the decompressed
// bytes are written back with mutations (truncated at many lengths, single
// bytes overwritten at many offsets) and parsed again: each must either
// parse or be refused with an exception, never read out of bounds.
//
// usage: parse_stress [--parse-only] <scratch dir> <model file>...
#include "../../katago_amd/host/neuralnet/desc.h"

#include <zlib.h>

#include <cstdio>
#include <exception>
#include <fstream>
#include <random>
#include <string>
#include <vector>

namespace {

std::string gunzip(const std::string& path) {
  gzFile f = gzopen(path.c_str(), "rb");
  if(f == nullptr) throw std::runtime_error("cannot open " + path);
  std::string out;
  char buf[1 << 16];
  int n;
  while((n = gzread(f, buf, sizeof(buf))) > 0) out.append(buf, n);
  gzclose(f);
  return out;
}

// 1: parsed, 0: refused with an exception.
int tryParse(const std::string& path) {
  try {
    ModelDesc desc;
    ModelDesc::loadFromFileMaybeGZipped(path, desc, "");
    return 1;
  }
  catch(const std::exception&) {
    return 0;
  }
}

}  // namespace

int main(int argc, char** argv) {
  int first = 1;
  const bool parseOnly = argc > 1 && std::string(argv[1]) == "--parse-only";
  if(parseOnly) first++;
  if(argc < first + 2) {
    std::fprintf(stderr, "usage: %s [--parse-only] <scratch dir> <model file>...\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[first];
  std::mt19937 rng(12345);
  long parsed = 0, refused = 0;
  for(int a = first + 1; a < argc; a++) {
    const std::string path = argv[a];
    {
      ModelDesc desc;
      ModelDesc::loadFromFileMaybeGZipped(path, desc, "");
      std::printf("%s: %s version %d\n", path.c_str(), desc.name.c_str(), desc.modelVersion);
    }
    if(parseOnly) continue;
    const bool text = path.find(".txt") != std::string::npos;
    const std::string raw = gunzip(path);
    const std::string out = dir + "/mutant" + (text ? ".txt" : ".bin");
    auto parseBytes = [&](const std::string& bytes) {
      std::ofstream(out, std::ios::binary).write(bytes.data(), (std::streamsize)bytes.size());
      if(tryParse(out)) parsed++;
      else refused++;
    };
    // Truncations: the first kilobyte byte-granular-ish, then spread over the file.
    for(size_t len : {size_t(0), size_t(1), size_t(7), size_t(40), size_t(200), size_t(1000)})
      if(len < raw.size()) parseBytes(raw.substr(0, len));
    for(int i = 1; i < 40; i++) parseBytes(raw.substr(0, raw.size() * i / 40));
    // Overwritten bytes: in the header (names, versions, dimensions) and anywhere.
    const size_t headerSpan = std::min(raw.size(), size_t(4096));
    for(int i = 0; i < 120; i++) {
      std::string m = raw;
      const size_t at = i < 80 ? rng() % headerSpan : rng() % raw.size();
      const char choices[] = {'0', '9', '-', ' ', '\n', 'x', '\0', '\xff'};
      m[at] = choices[rng() % sizeof(choices)];
      parseBytes(m);
    }
  }
  std::printf("mutants parsed %ld refused %ld\n", parsed, refused);
  std::printf("done\n");
  return 0;
}
