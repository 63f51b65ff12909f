// Model description and registry preflight (host only): what the library knows about a GGUF
// before any weight is read, and the checks a multi-model server runs before loading any.
#pragma once
#include <string>
#include <vector>

#include "gguf.h"

namespace lg {

struct ModelDesc {
  std::string name, family, architecture, release_date;
  std::vector<std::string> aliases;
};

// models::describe, src/models/mod.rs:32-64, plus the laya-decoder family ("ggmlc" with
// laya.model_name "laya-decoder", named by its general.name).  Throws LG_ERR_FORMAT with the
// reference's messages for anything else.
ModelDesc describe(const Gguf &g);

// The preflight of Registry::load, src/registry.rs:16-39: every path opened and described, every
// name and alias unique, the default known.  Returns the default's index.
int registry_preflight(const std::vector<std::string> &paths, const char *default_name);

}  // namespace lg
