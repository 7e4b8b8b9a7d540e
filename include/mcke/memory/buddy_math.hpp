// mcke/memory/buddy_math.hpp -- index arithmetic of a binary buddy tree over an
// arena of 2^arena_log2 bytes with blocks of at least 2^min_log2 bytes, as
// constexpr functions (the API of the reference's
// include/mcke/memory/buddy_math.hpp:81-207).
//
// Levels count down from the root: level 0 is the whole arena, level L holds
// 2^L blocks of 2^(arena_log2 - L) bytes.  Nodes are numbered in heap order
// (root 0, then each level left to right), so node i's children are 2i + 1 and
// 2i + 2, and a node and its buddy -- the other child of the same parent -- are
// an odd number and the even number after it.  BuddyAllocator reports a block's
// node number in this order as Allocation::block_id.
#pragma once

#include <bit>
#include <cstddef>

namespace mcke::buddy {

[[nodiscard]] constexpr bool is_power_of_two(std::size_t x) noexcept { return x && !(x & (x - 1)); }

// ceil(log2 x) for x >= 1 (0 for x <= 1).
[[nodiscard]] constexpr unsigned ceil_log2(std::size_t x) noexcept {
  return x <= 1 ? 0u : static_cast<unsigned>(std::bit_width(x - 1));
}

// floor(log2 x) for x >= 1 (0 for x == 0).
[[nodiscard]] constexpr unsigned floor_log2(std::size_t x) noexcept {
  return x ? static_cast<unsigned>(std::bit_width(x)) - 1u : 0u;
}

// x rounded up to a multiple of the power of two a.
[[nodiscard]] constexpr std::size_t align_up(std::size_t x, std::size_t a) noexcept {
  return (x + (a - 1)) & ~(a - 1);
}

// The deepest level, whose blocks are the minimum size.
[[nodiscard]] constexpr unsigned max_level(unsigned arena_log2, unsigned min_log2) noexcept {
  return arena_log2 - min_log2;
}

// Nodes in a tree of levels 0 .. max_lvl.
[[nodiscard]] constexpr std::size_t node_count(unsigned max_lvl) noexcept {
  return (std::size_t{2} << max_lvl) - 1;
}

[[nodiscard]] constexpr std::size_t block_bytes_at_level(unsigned arena_log2, unsigned level) noexcept {
  return std::size_t{1} << (arena_log2 - level);
}

[[nodiscard]] constexpr std::size_t nodes_at_level(unsigned level) noexcept { return std::size_t{1} << level; }

// The deepest level whose blocks hold `bytes` (requests below the minimum block
// take a minimum block); max_level + 1 when the request exceeds the arena.
[[nodiscard]] constexpr unsigned level_for_size(std::size_t bytes, unsigned arena_log2,
                                                unsigned min_log2) noexcept {
  const unsigned need = bytes <= (std::size_t{1} << min_log2) ? min_log2 : ceil_log2(bytes);
  return need > arena_log2 ? max_level(arena_log2, min_log2) + 1 : arena_log2 - need;
}

[[nodiscard]] constexpr std::size_t heap_index(unsigned level, std::size_t idx_in_level) noexcept {
  return nodes_at_level(level) - 1 + idx_in_level;
}

[[nodiscard]] constexpr unsigned level_of(std::size_t heap_idx) noexcept { return floor_log2(heap_idx + 1); }

[[nodiscard]] constexpr std::size_t index_in_level(std::size_t heap_idx) noexcept {
  return heap_idx + 1 - nodes_at_level(level_of(heap_idx));
}

[[nodiscard]] constexpr bool is_root(std::size_t heap_idx) noexcept { return heap_idx == 0; }

// Not for the root (check is_root first).
[[nodiscard]] constexpr std::size_t parent_of(std::size_t heap_idx) noexcept { return (heap_idx - 1) >> 1; }

[[nodiscard]] constexpr std::size_t left_child_of(std::size_t heap_idx) noexcept { return 2 * heap_idx + 1; }

[[nodiscard]] constexpr std::size_t right_child_of(std::size_t heap_idx) noexcept { return 2 * heap_idx + 2; }

// The other child of the same parent: odd nodes are left children, even ones
// right children.  Not for the root.
[[nodiscard]] constexpr std::size_t buddy_of(std::size_t heap_idx) noexcept {
  return (heap_idx & 1) ? heap_idx + 1 : heap_idx - 1;
}

// Byte offset of a node's block from the start of the arena.
[[nodiscard]] constexpr std::size_t offset_of(std::size_t heap_idx, unsigned arena_log2) noexcept {
  return index_in_level(heap_idx) * block_bytes_at_level(arena_log2, level_of(heap_idx));
}

// The node at `level` whose block holds byte `offset`.
[[nodiscard]] constexpr std::size_t node_at(std::size_t offset, unsigned level, unsigned arena_log2) noexcept {
  return heap_index(level, offset >> (arena_log2 - level));
}

static_assert(ceil_log2(1) == 0 && ceil_log2(2) == 1 && ceil_log2(3) == 2 && ceil_log2(257) == 9);
static_assert(floor_log2(1) == 0 && floor_log2(255) == 7 && floor_log2(256) == 8);
static_assert(heap_index(2, 3) == 6 && level_of(6) == 2 && index_in_level(6) == 3);
static_assert(buddy_of(5) == 6 && buddy_of(6) == 5 && parent_of(5) == parent_of(6));
static_assert(left_child_of(parent_of(5)) == 5 && right_child_of(parent_of(5)) == 6);
static_assert(offset_of(2, 20) == (std::size_t{1} << 19) && node_at(std::size_t{1} << 19, 1, 20) == 2);
static_assert(level_for_size(1, 20, 8) == 12 && level_for_size(300, 20, 8) == 11);
static_assert(level_for_size(std::size_t{1} << 20, 20, 8) == 0);
static_assert(level_for_size((std::size_t{1} << 20) + 1, 20, 8) == 13);

}  // namespace mcke::buddy
