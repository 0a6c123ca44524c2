// The QPACK_DEVICE=hip branch of load_model (/root/reference/src/model_llama.cpp:221-235), for a build that links the
// reference's own model_llama.cpp unchanged: there that file is compiled with -Dload_model=reference_load_model, and
// this load_model adds the branch in front of it.  In qpack itself the same lines go into load_model directly:
//
//   const bool hip = dev && !strcmp(dev, "hip");
//   if (arch == "llama" && hip) return make_llama_hip(c, max_ctx);
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>

#include "qpack/qpack.h"

namespace qp {

std::unique_ptr<Model> make_llama_hip(std::shared_ptr<Container> c, int max_ctx);
std::unique_ptr<Model> reference_load_model(const std::string &path, int max_ctx);

std::unique_ptr<Model> load_model(const std::string &path, int max_ctx) {
  const char *dev = getenv("QPACK_DEVICE");
  if (dev && !strcmp(dev, "hip")) {
    auto c = std::make_shared<Container>(path);
    if (c->config()["arch"].as_str() == "llama") return make_llama_hip(c, max_ctx);
    throw std::runtime_error("QPACK_DEVICE=hip: only Llama-family models are supported (arch='" + c->config()["arch"].as_str() + "')");
  }
  return reference_load_model(path, max_ctx);
}

}  // namespace qp
