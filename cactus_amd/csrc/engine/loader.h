// loader.h -- model folders of CACT tensor files to device memory
// (Model::init, cactus/engine/engine_model.cpp:47-55 and :72-160;
// Config::from_json, :403-520; QwenModel::load_weights_to_graph,
// cactus/models/model_qwen.cpp:17-49).
#pragma once

#include <string>

#include "cact_file.h"
#include "cactus_engine.h"

namespace cactus {

class QwenModel;

// Device copy of one CACT file: the data (INT4 stays packed) and its fp16
// group scales, allocated with cactus_hip_malloc; the caller frees both.
struct DeviceTensor {
    void* data = nullptr;
    void* scales = nullptr;
};
DeviceTensor upload_cact(const CactFile& f, void* stream);

// folder/config.txt in the reference's key=value form; keys it does not
// name keep the reference's defaults (engine.h:42-58).  Throws when the file
// is missing or describes a model this engine does not build.  group_size
// comes from the first layer's q projection file; max_seq is 0.
cactus_qwen_config read_qwen_config(const std::string& folder);

// Model::init(model_folder, context_size): reads the config and every tensor
// file of the Qwen3 layout, checks shapes, precisions and groups, uploads.
QwenModel* load_qwen_folder(const std::string& folder, size_t context_size);

}  // namespace cactus
