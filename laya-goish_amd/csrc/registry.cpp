// Model description and registry preflight (src/models/mod.rs:32-64, src/registry.rs:11-39).
#include "registry.h"

#include <map>
#include <memory>

#include "common.h"
#include "lg.h"

namespace lg {

ModelDesc describe(const Gguf &g) {
  ModelDesc d;
  d.architecture = g.str("general.architecture");
  if (d.architecture == "openthai_systemone") {
    d.name = d.family = "openthai-systemone";
    d.release_date = "2026-09-22";
    return d;
  }
  if (d.architecture == "ggmlc") {
    const std::string name = g.str("laya.model_name");
    if (name == "laya-decoder") {  // the synthetic decoder family; no reference counterpart
      const std::string gn = g.str("general.name");
      d.name = gn.empty() ? name : gn;
      d.family = name;
      return d;
    }
    if (name == "laya") d.family = "english";
    else if (name == "laya-multilingual") d.family = "multilingual";
    else if (name == "laya-typed-decisions") d.family = "typed-decisions";
    else fail(LG_ERR_FORMAT, "unsupported ggmlc model %s", name.c_str());
    d.name = name;
    d.aliases.push_back(d.family);
    if (d.family == "english") d.aliases.push_back("jev-latest");
    d.release_date = "2026-09-20";
    return d;
  }
  fail(LG_ERR_FORMAT, "unsupported GGUF architecture %s", d.architecture.c_str());
}

int registry_preflight(const std::vector<std::string> &paths, const char *default_name) {
  if (paths.empty()) fail(LG_ERR_INVALID, "at least one model is required");
  std::map<std::string, int> names;
  for (size_t i = 0; i < paths.size(); ++i) {
    std::unique_ptr<Gguf> g(Gguf::open_file(paths[i]));
    const ModelDesc d = describe(*g);
    std::vector<std::string> all{d.name};
    all.insert(all.end(), d.aliases.begin(), d.aliases.end());
    for (const std::string &n : all)
      if (!names.emplace(n, int(i)).second)
        fail(LG_ERR_INVALID, "duplicate model name or alias %s; load one checkpoint per model", n.c_str());
  }
  if (!default_name) return 0;
  auto it = names.find(default_name);
  if (it == names.end()) fail(LG_ERR_INVALID, "unknown default model %s", default_name);
  return it->second;
}

}  // namespace lg
