// The debugging library: the same C ABI with the engine on host threads. Tests load it to follow
// a match tick by tick; the package never loads it.
#include "runtime.h"

namespace eng {
namespace host {
std::unique_ptr<Device> MakeLibraryDevice(int threads) { return MakeHostDevice(threads); }
extern const char *const kBackendName = "host";
}  // namespace host
}  // namespace eng

#include <sstream>

// The field layout of a state, one line per field: byte position, size and path. Tests use it to
// name the first field where two states differ.
extern "C" __attribute__((visibility("default"))) const char *cuju_debug_state_schema(const char *bytes, unsigned long long size) {
    thread_local std::string text;
    try {
        std::string in(bytes, size);
        auto w = std::make_unique<eng::World>();
        eng::host::StateCodec codec;
        if (!codec.Load(in, *w)) return nullptr;
        std::vector<eng::codec::SchemaEntry> schema;
        codec.Save(*w, &schema);
        std::ostringstream o;
        for (const auto &e : schema) o << e.position << ' ' << e.size << ' ' << e.path << '\n';
        text = o.str();
        return text.c_str();
    } catch (...) {
        return nullptr;
    }
}
