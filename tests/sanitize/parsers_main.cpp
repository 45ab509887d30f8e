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
//   pack:<file>     a request as JSON {"first", "resident", "align", "rows",
//                   "groups": [{"prefix": [...], "branches": [{"tokens":
//                   [...], "want": [...]}]}]}: pack_groups (engine.rs:
//                   1512-1571), then align_groups; every wanted and decoded
//                   row of the aligned layout must lie inside it (a decoded
//                   row may equal its end: a group with no tokens)
#include <cstdio>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "json.h"
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
    } else if (kind == "pack") {
        const std::vector<uint8_t> b = bytes_of(path);
        const omg::Json req = omg::Json::parse(std::string(b.begin(), b.end()));
        const omg::Json& gs = req["groups"];
        std::vector<std::vector<uint32_t>> prefixes, tokens, wants;
        std::vector<std::vector<omg::BranchIn>> branches(gs.arr.size());
        std::vector<omg::GroupIn> groups;
        auto ints = [](const omg::Json& a) {
            std::vector<uint32_t> v;
            for (const omg::Json& x : a.arr) v.push_back(uint32_t(x.u64(0)));
            return v;
        };
        prefixes.reserve(gs.arr.size());
        size_t nb = 0;
        for (const omg::Json& g : gs.arr) nb += g["branches"].arr.size();
        tokens.reserve(nb);
        wants.reserve(nb);
        for (size_t gi = 0; gi < gs.arr.size(); ++gi) {
            const omg::Json& g = gs.arr[gi];
            prefixes.push_back(ints(g["prefix"]));
            for (const omg::Json& br : g["branches"].arr) {
                tokens.push_back(ints(br["tokens"]));
                wants.push_back(ints(br["want"]));
                branches[gi].push_back(omg::BranchIn{tokens.back().data(), int64_t(tokens.back().size()),
                                                     wants.back().data(), int64_t(wants.back().size())});
            }
            groups.push_back(omg::GroupIn{prefixes.back().data(), int64_t(prefixes.back().size()),
                                          branches[gi].data(), int64_t(branches[gi].size())});
        }
        const int64_t first = int64_t(req["first"].u64(0));
        if (first >= int64_t(groups.size())) omg::fail(omg::E_INVALID, "first group out of range");
        const omg::Packed pk = omg::pack_groups(groups.data(), int64_t(groups.size()), first,
                                                req["resident"].boolean(false));
        const omg::Packed al = omg::align_groups(pk, int64_t(req["align"].u64(1)), int64_t(req["rows"].u64(1 << 20)));
        for (const auto& w : al.wanted)
            if (w[3] < 0 || w[3] >= int64_t(al.ids.size())) omg::fail(omg::E_INVALID, "wanted row outside the pass");
        for (const auto& d : al.decoded)
            if (d.second < al.base || d.second > al.total) omg::fail(omg::E_INVALID, "decoded row outside the pass");
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
