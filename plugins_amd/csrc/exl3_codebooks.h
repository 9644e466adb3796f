// exl3_codebooks.h -- the table codebooks a pack may name (spec1, std1,
// pair1): the shipped constant tables and the resolution of a quantization
// block's `codebook_table` / `codebook_digest` against them
// (sushi_ds41/src/sushi/exl3/codebook_tables.zig:99-104,266-279).
#pragma once

#include <stdint.h>

#include "exl3_json.h"

namespace exl3 {

// Codebooks as the pack format numbers them (sushi_ds41/src/sushi/exl3/
// expert_exl3.zig:54-60).
enum PackCodebook { PACK_MUL1 = 0, PACK_MCG = 1, PACK_SPEC1 = 2, PACK_PAIR1 = 3, PACK_STD1 = 4 };

// One shipped table: rows for every even rate n from n_lo, each row
// {mult, mask} (spec1, std1) or {mult, rot, mask0, mask1} (pair1), the
// fields the reference orders them in.
struct CodebookTable {
  const char *name;
  int codebook;  // PackCodebook
  int window;    // the window it was searched at (pair1 holds only there)
  const char *digest;
  const char *superseded;  // an earlier version's digest, refused as legacy ("" none)
  int n_lo;
  int rows;
  const uint32_t (*data)[4];
};

// The pack codebook a name denotes, -1 for anything else.
int pack_codebook_of(const char *name);

// The table `block` names for `codebook` (spec1, std1 or pair1) at `window`.
// Returns nullptr and sets *out on success, else the refusal's text, the
// library's prefix and the reference's name (codebook_tables.zig:21-29:
// Exl3CodebookTableUnknown, ...DigestMismatch, ...LegacyConfig,
// ...CodebookMismatch, ...WindowMismatch), a static string.
const char *resolve_codebook_table(const Json &block, int codebook, int window,
                                   const CodebookTable **out);

// The table's row for rate n in the kernels' order {mult, mask0, mask1, rot}
// (hash-mask rows: {mult, mask, 0, 0}); false when it has none
// (codebook_tables.zig:48-52).
bool codebook_row(const CodebookTable &t, int n, uint32_t row[4]);

}  // namespace exl3
