#pragma once

// Logical spatial tiles of one latent frame: fixed runs of `tile_tokens`
// consecutive (row-major) tokens, the last run possibly shorter. Tile ids are
// stable across frames, so tile t of frame f covers token rows
// f*tokens_per_frame + [tile_start(t), tile_start(t) + tile_count(t)).
//
// Replaces the reference struct of the same name
// (reference: src/tile_layout.h:13-31); member names and arithmetic are kept
// because callers (driver, ctypes tests) depend on them.
//   1560 tokens / 16  -> 98 tiles, last tile 8 tokens
//   3600 tokens / 16  -> 225 tiles, all full

struct TileLayout {
    int tokens_per_frame;
    int tile_tokens;
    int tiles_per_frame;

    TileLayout(int tpf, int tt)
        : tokens_per_frame(tpf), tile_tokens(tt),
          tiles_per_frame(tt > 0 ? (tpf + tt - 1) / tt : 0) {}

    long tile_start(long tile_id) const { return tile_id * (long)tile_tokens; }

    int tile_count(long tile_id) const {
        const long left = (long)tokens_per_frame - tile_start(tile_id);
        return (int)(left < (long)tile_tokens ? left : (long)tile_tokens);
    }

    long tile_of_token(long token) const { return token / tile_tokens; }
};
