// Weights from the converter's safetensors files (src/weights.rs): the file is
// memory-mapped, its JSON header parsed and checked (the `format` metadata
// tag, offsets inside the file, dtype sizes, alignment), and every tensor the
// model asks for is checked against its expected shape before the device
// loaders (WeightStore) copy it to HBM. Host code only.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "unet.hpp"

namespace mh {

// src/weights.rs:18
constexpr const char *kWeightsFormat = "moebius-cpu/1";

struct FileTensor {
    uint32_t dtype = 0;  // kF32 / kF16
    std::vector<int64_t> shape;
    const void *data = nullptr;  // inside the mapping
    int64_t numel = 0;
};

class WeightsFile {
  public:
    // src/weights.rs:40-72: opens and maps `path`; the format tag must equal
    // `expected_format`. Errors: kIo (cannot open / map), kWeights (malformed
    // header, wrong format, bad offsets or dtypes).
    WeightsFile(const std::string &path, const std::string &expected_format = kWeightsFormat);
    ~WeightsFile();
    WeightsFile(const WeightsFile &) = delete;
    WeightsFile &operator=(const WeightsFile &) = delete;
    const std::string *metadata(const std::string &key) const;
    const FileTensor *find(const std::string &name) const;
    const std::map<std::string, FileTensor> &tensors() const { return tensors_; }
    const std::string &path() const { return path_; }

  private:
    std::string path_;
    void *map_ = nullptr;
    size_t size_ = 0;
    std::map<std::string, FileTensor> tensors_;
    std::map<std::string, std::string> meta_;
};

enum class ModelKind : uint32_t { UNet = 0, Vae = 1 };

// The converted tensor set each model loads (names and shapes after
// tools/convert_weights.py:13-33), from the architecture of src/config.rs.
std::map<std::string, std::vector<int64_t>> expected_tensors(ModelKind kind);

// The tensors of `kind` from an open file, shape-checked (src/weights.rs:84-96:
// a missing tensor or another shape is kWeights); for the VAE also the
// `scaling_factor` metadata (src/vae/mod.rs:88-93). The NamedTensors point into
// the mapping: keep `f` open while they are used.
std::vector<NamedTensor> model_tensors(const WeightsFile &f, ModelKind kind);

}  // namespace mh
