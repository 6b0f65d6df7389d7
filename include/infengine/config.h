// C++ spelling of the engine's shape constants (reference: config.h:5-27).
#pragma once
#include <string>
#include <vector>

#include "../infengine.h"

namespace InfEngineConfig {
static const std::string TOKENIZER_PATH = "models/llama_3.1_8b/tokenizer.json";
static const int MAX_CONTEXT_LENGTH = IE_MAX_CONTEXT_LENGTH;
static const int VOCAB_SIZE = IE_VOCAB_SIZE;

static const int NUM_LAYERS = IE_NUM_LAYERS;
static const int HIDDEN_SIZE = IE_HIDDEN_SIZE;

static const int NUM_Q_HEADS = IE_NUM_Q_HEADS;
static const int NUM_KV_HEADS = IE_NUM_KV_HEADS;

static const int HEAD_DIM = IE_HEAD_DIM;
static const int FFN_DIM = IE_FFN_DIM;

// Bytes per stored activation / weight element (bf16 here; fp16 in the reference).
static const int HALF_SIZE = IE_BF16_SIZE;

static const std::vector<std::string> MODEL_FILES = {
    "models/llama_3.1_8b/model-00001-of-00004.safetensors",
    "models/llama_3.1_8b/model-00002-of-00004.safetensors",
    "models/llama_3.1_8b/model-00003-of-00004.safetensors",
    "models/llama_3.1_8b/model-00004-of-00004.safetensors"};
}  // namespace InfEngineConfig
