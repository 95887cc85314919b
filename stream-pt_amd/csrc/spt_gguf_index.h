// GGUF tensor directory (host side): the index ggufindex.Open builds
// (ggufindex/index.go:60-234) -- headers, metadata value ranges, tensor
// directories and the per-layer grouping of one model split over one or more
// files -- from which the path's tensors are uploaded to HBM unchanged.
#pragma once

#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace spt {
namespace gguf {

// ggufindex.Range (index.go:15-19), the file as an index into Model::paths.
struct Range {
    int file = 0;
    uint64_t start = 0, end = 0;
};

// ggufindex.Tensor (index.go:21-26); layer = N of a "blk.N." name, else -1.
struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> shape;
    Range range;
    int64_t layer = -1;
};

// ggufindex.MetadataValue (metadata.go:13-17): the encoded value's range.
struct MetaValue {
    uint32_t type = 0;
    Range range;
};

// ggufindex.Model (index.go:38-47): layers in order 0..layer_count-1, each
// with its tensors sorted by name and its spans (one per file, sorted by
// path); the tensors outside the layers sorted by name.
struct Model {
    std::vector<std::string> paths;
    int64_t layer_count = 0;
    std::vector<std::vector<Tensor>> layers;
    std::vector<std::vector<Range>> spans;
    std::vector<Tensor> shared;
    uint64_t alignment = 0;
    std::map<std::string, MetaValue> metadata;
};

// ggufindex.Open; on failure *err holds the reference's message.
bool open(const std::vector<std::string> &paths, Model *model, std::string *err);

// tensorSize (index.go:535-574): the byte size of a tensor of GGML type
// `type` and this shape, or false with *err set.
bool tensor_size(uint32_t type, const std::vector<uint64_t> &shape, uint64_t *bytes, std::string *err);

// TensorByName (index.go:577-591): the tensors outside the layers first,
// then the layers in order.
const Tensor *find(const Model &m, const std::string &name);

}  // namespace gguf
}  // namespace spt
