// CPU harness of the engine's parsers of untrusted bytes, built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_sanitize.py
// (g++ on grande_amd/csrc/{model,gguf,state}.cpp and this file; no device
// code).  Each argument is `<kind>:<path>`; each input is parsed and
// either accepted or refused with omg::Error, one line per input on stdout.
// An out-of-bounds read, overflow or other undefined behaviour aborts the
// process with the sanitizer's report instead.
//   config:<file>   Config::from_json + validate (model.rs:66-254)
//   gguf:<file>     load_gguf (tools/export_wgpu_gguf.py's layout)
//   dir:<path>      load_dir (config.json + manifest.json + *.bin)
//   state:<file>    SavedState::from_bytes for model id "m", then to_bytes
//                   must reproduce the input (engine.rs:517-579)
#include <cstdio>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "model.h"
#include "state.h"

static std::vector<uint8_t> bytes_of(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

static void run(const std::string& kind, const std::string& path) {
    if (kind == "config") {
        const std::vector<uint8_t> b = bytes_of(path);
        omg::Config::from_json(omg::Json::parse(std::string(b.begin(), b.end()))).validate();
    } else if (kind == "gguf") {
        omg::Weights w = omg::load_gguf(path);
        w.config.validate();
    } else if (kind == "dir") {
        omg::load_dir(path);
    } else if (kind == "state") {
        const std::vector<uint8_t> b = bytes_of(path);
        const omg::SavedState s = omg::SavedState::from_bytes(b.data(), b.size(), "m");
        const std::vector<uint8_t> again = s.to_bytes("m");
        // from_bytes may stop before trailing bytes; what it read re-encodes exactly
        if (again.size() > b.size() || !std::equal(again.begin(), again.end(), b.begin()))
            omg::fail(omg::E_STATE, "re-encoded bytes differ from the input");
    } else {
        omg::fail(omg::E_INVALID, "unknown kind " + kind);
    }
}

int main(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        const size_t colon = arg.find(':');
        if (colon == std::string::npos) return 2;
        const std::string kind = arg.substr(0, colon), path = arg.substr(colon + 1);
        try {
            run(kind, path);
            std::printf("ok %s\n", path.c_str());
        } catch (const omg::Error& e) {
            std::printf("refused %s: %s\n", path.c_str(), e.what());
        }
    }
    return 0;
}
