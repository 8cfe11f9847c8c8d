// policy_experiment: command-line driver with the reference driver's flag set
// and output lines (reference: src/run_policy_experiment.cu:71-317), so
// scripts written for the reference binary can drive this one.
//
//   --policy none|uniform|recency|motion|reuse_weighted
//   --attn-mode intra|cross   --streaming
//   --q --k --v FILE          flat fp32 [frames*tokens*hidden] (.bin)
//   --motion-csv FILE         frame_id,tile_id,motion_score,is_static,
//                             token_start,token_count[,reuse]
//   --out FILE                flat fp32 output
//   --frames --tokens --hidden --heads --tile-tokens --set-aside-bytes
// Additive flags: --dtype fp32|bf16 (bf16: inputs rounded to bf16 on the
// host, output widened back to fp32 for the file), --window W (sliding
// window of W frames in cross mode).
//
// Host side only: device work goes through libkvpersist.so's C-ABI.

#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "kvp_c_api.h"
#include "tile_gating_policy.h"

namespace {

void die(const char* what) {
    fprintf(stderr, "FAIL %s: %s\n", what, kvp_last_error());
    exit(1);
}

std::vector<float> read_bin(const std::string& path, size_t elems, const char* what) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s (%s)\n", path.c_str(), what);
        exit(1);
    }
    std::vector<float> buf(elems);
    if (fread(buf.data(), sizeof(float), elems, f) != elems) {
        fprintf(stderr, "short read on %s\n", path.c_str());
        exit(1);
    }
    fclose(f);
    return buf;
}

// Rows without a matching (frame, tile) keep score 0, as in the reference.
std::vector<float> read_motion_csv(const std::string& path, int frames, int num_tiles) {
    FILE* f = fopen(path.c_str(), "r");
    if (!f) {
        fprintf(stderr, "cannot open motion csv %s\n", path.c_str());
        exit(1);
    }
    std::vector<float> scores((size_t)frames * num_tiles, 0.f);
    char line[256];
    if (!fgets(line, sizeof line, f)) {
        fclose(f);
        return scores;
    }
    while (fgets(line, sizeof line, f)) {
        int fr, tid, is_static, start, count, reuse = 0;
        float score;
        const int got = sscanf(line, "%d,%d,%f,%d,%d,%d,%d", &fr, &tid, &score, &is_static,
                               &start, &count, &reuse);
        if ((got == 6 || got == 7) && fr >= 0 && fr < frames && tid >= 0 && tid < num_tiles)
            scores[(size_t)fr * num_tiles + tid] = score;
    }
    fclose(f);
    return scores;
}

uint16_t to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN stays NaN
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
    return (uint16_t)(u >> 16);
}

float from_bf16(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float x;
    memcpy(&x, &u, 4);
    return x;
}

void make_parent_dirs(const std::string& path) {
    for (size_t i = 1; i < path.size(); ++i) {
        if (path[i] == '/') {
            std::string d = path.substr(0, i);
            if (mkdir(d.c_str(), 0755) != 0 && errno != EEXIST) return;
        }
    }
}

// Command-line options. The flag names, meanings and defaults are the
// reference driver's (src/run_policy_experiment.cu:77-95), so its scripts can
// drive this binary; --dtype and --window are additions.
struct Options {
    std::string policy, attn_mode = "intra", q, k, v, motion_csv, out, dtype = "fp32";
    int streaming = 0, window = 0;
    long frames = 8, tokens = 1560, hidden = 1536, heads = 12;
    long tile_tokens = 16, set_aside = 2162688;
};

// One table entry per flag, with exactly one target; `--streaming` is a
// switch, every other flag takes the next argument.
struct FlagSpec {
    const char* name;
    std::string* text;
    long* number;
    int* flag;
    bool is_switch;
};

bool parse_options(int argc, char** argv, Options& o) {
    const FlagSpec table[] = {
        {"--policy", &o.policy, nullptr, nullptr, false},
        {"--attn-mode", &o.attn_mode, nullptr, nullptr, false},
        {"--streaming", nullptr, nullptr, &o.streaming, true},
        {"--q", &o.q, nullptr, nullptr, false},
        {"--k", &o.k, nullptr, nullptr, false},
        {"--v", &o.v, nullptr, nullptr, false},
        {"--motion-csv", &o.motion_csv, nullptr, nullptr, false},
        {"--out", &o.out, nullptr, nullptr, false},
        {"--frames", nullptr, &o.frames, nullptr, false},
        {"--tokens", nullptr, &o.tokens, nullptr, false},
        {"--hidden", nullptr, &o.hidden, nullptr, false},
        {"--heads", nullptr, &o.heads, nullptr, false},
        {"--tile-tokens", nullptr, &o.tile_tokens, nullptr, false},
        {"--set-aside-bytes", nullptr, &o.set_aside, nullptr, false},
        {"--dtype", &o.dtype, nullptr, nullptr, false},
        {"--window", nullptr, nullptr, &o.window, false},
    };
    for (int i = 1; i < argc; ++i) {
        const FlagSpec* spec = nullptr;
        for (const FlagSpec& f : table)
            if (strcmp(argv[i], f.name) == 0) spec = &f;
        if (!spec) {
            fprintf(stderr, "unknown arg %s\n", argv[i]);
            return false;
        }
        if (spec->is_switch) {
            *spec->flag = 1;
            continue;
        }
        if (i + 1 >= argc) {
            fprintf(stderr, "missing value for %s\n", spec->name);
            return false;
        }
        const char* value = argv[++i];
        if (spec->text) {
            *spec->text = value;
            continue;
        }
        char* end = nullptr;
        errno = 0;
        const long n = strtol(value, &end, 10);
        if (errno != 0 || end == value || *end != '\0') {
            fprintf(stderr, "%s needs an integer, got '%s'\n", spec->name, value);
            return false;
        }
        if (spec->number)
            *spec->number = n;
        else
            *spec->flag = (int)n;
    }
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    Options opt;
    if (!parse_options(argc, argv, opt)) return 1;
    const std::string& policy_name = opt.policy;
    const std::string &q_path = opt.q, &k_path = opt.k, &v_path = opt.v;
    const std::string &csv_path = opt.motion_csv, &out_path = opt.out;
    const std::string &attn_mode = opt.attn_mode, &dtype_name = opt.dtype;
    const int streaming = opt.streaming, window = opt.window;
    const long frames = opt.frames, tokens = opt.tokens, hidden = opt.hidden, heads = opt.heads;
    const long tile_tokens = opt.tile_tokens, set_aside = opt.set_aside;
    const bool xframe = attn_mode == "cross";
    const int dtype = dtype_name == "bf16" ? 1 : 0;
    if (dtype_name != "bf16" && dtype_name != "fp32") {
        fprintf(stderr, "unknown dtype %s\n", dtype_name.c_str());
        return 1;
    }
    const long num_tiles = (tokens + tile_tokens - 1) / tile_tokens;
    const size_t elems = (size_t)frames * tokens * hidden;

    TileGatingPolicy* probe = make_tile_gating_policy(policy_name.c_str(), (int)num_tiles,
                                                      (int)frames);
    if (!probe) {
        fprintf(stderr, "unknown policy %s\n", policy_name.c_str());
        return 1;
    }
    delete probe;
    const bool persist = policy_name != "none";

    std::vector<float> h_q = read_bin(q_path, elems, "q");
    std::vector<float> h_k = read_bin(k_path, elems, "k");
    std::vector<float> h_v = read_bin(v_path, elems, "v");
    std::vector<float> scores;
    if (persist) scores = read_motion_csv(csv_path, (int)frames, (int)num_tiles);

    const size_t esz = dtype == 1 ? 2 : 4;
    void* d_q = kvp_dev_alloc(elems * esz);
    void* d_k = kvp_dev_alloc(elems * esz);
    void* d_v = kvp_dev_alloc(elems * esz);
    void* d_out = kvp_dev_alloc(elems * esz);
    if (!d_q || !d_k || !d_v || !d_out) die("device alloc");
    auto upload = [&](void* dst, const std::vector<float>& src) {
        if (dtype == 1) {
            std::vector<uint16_t> tmp(src.size());
            for (size_t i = 0; i < src.size(); ++i) tmp[i] = to_bf16(src[i]);
            if (kvp_memcpy_h2d(dst, tmp.data(), tmp.size() * 2, nullptr)) die("H2D");
        } else {
            if (kvp_memcpy_h2d(dst, src.data(), src.size() * 4, nullptr)) die("H2D");
        }
    };
    upload(d_q, h_q);
    upload(d_k, h_k);
    upload(d_v, h_v);

    void* pl = kvp_pipeline_create(policy_name.c_str(), xframe ? 1 : 0, streaming, (int)frames,
                                   (int)tokens, (int)hidden, (int)heads, (int)tile_tokens,
                                   persist ? set_aside : 0, dtype, window, 0);
    if (!pl) {
        fprintf(stderr, "manager init failed: %s\n", kvp_last_error());
        return 1;
    }
    if (persist) {
        const size_t tile_bytes = (size_t)tile_tokens * hidden * esz * 2;
        printf("policy=%s slots=%ld tile_bytes=%zu set_aside=%ld\n", policy_name.c_str(),
               kvp_pipeline_slots(pl), tile_bytes, set_aside);
    }
    std::vector<long> ids((size_t)frames * num_tiles + 64);
    for (int f = 0; f < (int)frames; ++f) {
        if (kvp_pipeline_step(pl, f, d_q, d_k, d_v, d_out, persist ? scores.data() : nullptr))
            die("frame step");
        if (persist && f == 0) {
            const int count = kvp_pipeline_selected(pl, ids.data(), (int)ids.size());
            printf("frame 0 selected tiles:");
            for (int i = 0; i < count; ++i) {
                const long gid = ids[i];
                const long sf = xframe ? gid / num_tiles : f;
                const long tl = xframe ? gid % num_tiles : gid;
                const float sc = (sf < frames && tl < num_tiles) ? scores[sf * num_tiles + tl] : 0.f;
                printf(" %ld(f%ld,t%ld,score %.3f)", gid, sf, tl, sc);
            }
            printf("\n");
        }
    }
    if (kvp_device_sync()) die("run");
    if (persist && streaming) printf("streamed staged_bytes=%ld\n", kvp_pipeline_staged_bytes(pl));

    std::vector<float> h_out(elems);
    if (dtype == 1) {
        std::vector<uint16_t> tmp(elems);
        if (kvp_memcpy_d2h(tmp.data(), d_out, elems * 2, nullptr)) die("D2H out");
        for (size_t i = 0; i < elems; ++i) h_out[i] = from_bf16(tmp[i]);
    } else {
        if (kvp_memcpy_d2h(h_out.data(), d_out, elems * 4, nullptr)) die("D2H out");
    }
    make_parent_dirs(out_path);
    FILE* fo = fopen(out_path.c_str(), "wb");
    if (!fo) {
        fprintf(stderr, "cannot open %s for write\n", out_path.c_str());
        return 1;
    }
    fwrite(h_out.data(), 4, elems, fo);
    fclose(fo);
    printf("policy=%s -> %s (%zu bytes)\n", policy_name.c_str(), out_path.c_str(), elems * 4);

    kvp_pipeline_destroy(pl);
    kvp_dev_free(d_q);
    kvp_dev_free(d_k);
    kvp_dev_free(d_v);
    kvp_dev_free(d_out);
    return 0;
}
