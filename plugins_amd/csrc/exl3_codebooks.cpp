// exl3_codebooks.cpp -- the shipped codebook tables and their resolution.
// The constants are the pack contract's (sushi_ds41/src/sushi/exl3/
// codebook_tables.zig:99-206 and expert_exl3.zig:23-46); the GPU decode
// tests compare every row's decode with the oracle's copy, which the
// tables' published digests pin.
#include "exl3_codebooks.h"

#include <cstring>
#include <string>

namespace exl3 {
namespace {

// pair1-w16-v1 at n = 24..64: {mult, rot, mask0, mask1}.
const uint32_t kPair1[21][4] = {
    {0x58F41BF3u, 3, 0x8ED78C13u, 0x8EEE8C03u},  {0x58F41BF3u, 3, 0x8ED78C13u, 0x8EEE8C03u},
    {0x7AA2BE15u, 3, 0x8ED78C13u, 0x8ECE8C03u},  {0x7B229E11u, 3, 0x8ED78C13u, 0x8ECE8C03u},
    {0x3B22BE15u, 3, 0x8ED78C13u, 0x8ECE8C03u},  {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu},
    {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu}, {0x46C63E17u, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0x82439F67u, 19, 0x8E6E8F9Au, 0x8E258FAEu}, {0xE2C7FC0Du, 19, 0x8F408FB0u, 0x8F918F89u},
    {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u}, {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u},
    {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u},
};

// spec1-w15 at n = 16..128: {mult, mask}.
const uint32_t kSpec1W15[57][4] = {
    {0x84d1cf89u, 0x8fe08947u}, {0x84c1cf49u, 0x8fe48a47u}, {0x84d1cfe9u, 0x8fe08a47u},
    {0x84d1cfc9u, 0x8ff08b67u}, {0x84c1cf49u, 0x8fe08b47u}, {0x84c1cf99u, 0x8fa08b66u},
    {0x862c1d37u, 0x8ff28c50u}, {0x84641fb7u, 0x8fa08c40u}, {0x846c1fa7u, 0x8fe08c80u},
    {0x844c1fd7u, 0x8ffe8c98u}, {0x846c1fa7u, 0x8ffe8d10u}, {0x845c1f77u, 0x8ffa8e10u},
    {0x843c1fa7u, 0x8ffe8e40u}, {0x843c1fa7u, 0x8ffe8e40u}, {0x842c1fc7u, 0x8fff8f00u},
    {0x843c1fb7u, 0x8ffe8f10u}, {0x84181fb5u, 0x8fe08f80u}, {0x84081f75u, 0x8ffa8f72u},
    {0x84081f75u, 0x8fd68fd0u}, {0x84241f27u, 0x8ffc8fc0u}, {0x84081f73u, 0x8fe08f80u},
    {0x84081f75u, 0x8fbe8ff0u}, {0x3fed4cefu, 0x8fe08fe0u}, {0x3fed4cefu, 0x8fc18ff2u},
    {0x3fed4cefu, 0x8ff08ff0u}, {0x3fed4cefu, 0x8fe28ff0u}, {0x3fed4cefu, 0x8fe08fe0u},
    {0x80081b7bu, 0x8ff08fc8u}, {0x80081b7bu, 0x8ff48fc0u}, {0x400036cbu, 0x8f448fffu},
    {0x400036cbu, 0x8fe48fffu}, {0x400036cbu, 0x8f448ff9u}, {0x8000387bu, 0x8fe08ff7u},
    {0x8000387bu, 0x8fc08feeu}, {0x80003779u, 0x8fe88ffeu}, {0x80003779u, 0x8fc88ffcu},
    {0x80003779u, 0x8fca8ffcu}, {0x80003779u, 0x8fcc8ffeu}, {0x80003879u, 0x8ffc8fefu},
    {0x50003851u, 0x8ff98fffu}, {0xd0003751u, 0x8ff98fffu}, {0x50003851u, 0x8ff98ff6u},
    {0xd0003931u, 0x8ff98fffu}, {0xd0003931u, 0x8ff98ffau}, {0xd0003931u, 0x8ff48ffau},
    {0x300031b1u, 0x8ffb8ffcu}, {0x300031b1u, 0x8ffa8ffeu}, {0x300031b1u, 0x8ffb8ffcu},
    {0xc00031f1u, 0x8ffe8ffau}, {0x400031f1u, 0x8ffe8ffeu}, {0x400031f1u, 0x8ffe8ffeu},
    {0x40003931u, 0x8ffc8ffcu}, {0x40003931u, 0x8ffc8ffcu}, {0x40003931u, 0x8ff88ffeu},
    {0x40003931u, 0x8ff88ffcu}, {0x80003811u, 0x8ffc8ffcu}, {0x80003811u, 0x8ffc8ffcu},
};

// spec1-w16 at n = 24..64: {mult, mask}.
const uint32_t kSpec1W16[21][4] = {
    {0x862d1c19u, 0x8fee8c30u}, {0x862d1d37u, 0x8fee8c30u}, {0x862d1d37u, 0x8ffe8c10u},
    {0x842f1f37u, 0x8ffc8d10u}, {0x840f1f67u, 0x8ffc8d10u}, {0x844f1f77u, 0x8ffe8d40u},
    {0x840d1f37u, 0x8ffe8e10u}, {0x84091f33u, 0x8fe88e00u}, {0x844d1f77u, 0x8fe08e00u},
    {0x843c1fa7u, 0x8ffe8e40u}, {0x844c1f7fu, 0x8ffc8f02u}, {0x841c1fb9u, 0x8fe88f04u},
    {0x842c1fc7u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8ffe8fc1u},
    {0x83fc1fa3u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8fee8fc0u}, {0x84061f77u, 0x8fd08f80u},
    {0x84081f6fu, 0x8ffe8fc0u}, {0x84081f25u, 0x8ffe8fe0u}, {0x83f81f6fu, 0x8ff48fc0u},
};

// std1: one pair at every rate n = 24..64.
#define EXL3_STD1_ROW {0x840C1F37u, 0x8FFE8FD0u, 0u, 0u}
const uint32_t kStd1[21][4] = {
    EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW,
    EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW,
    EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW,
    EXL3_STD1_ROW, EXL3_STD1_ROW, EXL3_STD1_ROW,
};
#undef EXL3_STD1_ROW

const CodebookTable kTables[] = {
    {"pair1-w16-v1", PACK_PAIR1, 16, "c089b4eb", "", 24, 21, kPair1},
    {"spec1-w15", PACK_SPEC1, 15, "37f72431", "2ac2594d", 16, 57, kSpec1W15},
    {"spec1-w16", PACK_SPEC1, 16, "753ffa03", "", 24, 21, kSpec1W16},
    {"std1", PACK_STD1, 15, "c5dba171", "", 24, 21, kStd1},
};

}  // namespace

int pack_codebook_of(const char *name) {
  static const char *names[] = {"mul1", "mcg", "spec1", "pair1", "std1"};
  for (int i = 0; i < 5; ++i)
    if (std::strcmp(name, names[i]) == 0) return i;
  return -1;
}

const char *resolve_codebook_table(const Json &block, int codebook, int window,
                                   const CodebookTable **out) {
  if (codebook != PACK_SPEC1 && codebook != PACK_STD1 && codebook != PACK_PAIR1)
    return "turboexl3_mi355x: Exl3CodebookTableCodebookMismatch";
  const Json *name = block.get("codebook_table");
  if (!name || name->kind != Json::STRING) return "turboexl3_mi355x: Exl3CodebookTableUnknown";
  const CodebookTable *t = nullptr;
  for (const CodebookTable &c : kTables)
    if (name->str == c.name) t = &c;
  if (!t) return "turboexl3_mi355x: Exl3CodebookTableUnknown";
  const Json *digest = block.get("codebook_digest");
  if (!digest || digest->kind != Json::STRING) return "turboexl3_mi355x: Exl3CodebookTableDigestMismatch";
  if (t->superseded[0] && digest->str == t->superseded) return "turboexl3_mi355x: Exl3CodebookTableLegacyConfig";
  if (digest->str != t->digest) return "turboexl3_mi355x: Exl3CodebookTableDigestMismatch";
  if (t->codebook != codebook) return "turboexl3_mi355x: Exl3CodebookTableCodebookMismatch";
  // spec1 and std1 rows decode at any window; pair1's only at its own
  if (t->codebook == PACK_PAIR1 && t->window != window) return "turboexl3_mi355x: Exl3CodebookTableWindowMismatch";
  *out = t;
  return nullptr;
}

bool codebook_row(const CodebookTable &t, int n, uint32_t row[4]) {
  if (n % 2 != 0 || n < t.n_lo || (n - t.n_lo) / 2 >= t.rows) return false;
  const uint32_t *r = t.data[(n - t.n_lo) / 2];
  if (t.codebook == PACK_PAIR1) {
    row[0] = r[0];
    row[1] = r[2];
    row[2] = r[3];
    row[3] = r[1];
  } else {
    row[0] = r[0];
    row[1] = r[1];
    row[2] = 0;
    row[3] = 0;
  }
  return true;
}

}  // namespace exl3
