// Canonical-Huffman stream format constants shared by the device kernels
// (cbq_huffman.hip) and the host table builders and indexer
// (cbq_huff_host.cpp).
#pragma once

namespace cbq_huff {

constexpr int kLutBits = 12;                        // first-level table: 12 stream bits
constexpr int kLutSize = 1 << kLutBits;
constexpr int kChunk = 4096;                        // symbols per chunk (chunk_off entry)
constexpr int kSub = 64;                            // symbols per sub-block (sub_len entry)
constexpr int kMaxLen = 32;                         // longest code the format allows
constexpr int kCanonInts = 3 * (kMaxLen + 1) + 1;   // first | count | base | invalid payload

}  // namespace cbq_huff
