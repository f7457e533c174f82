"""Writes kv_append_kats.json: the page-append cases of mini-vllm-rs's own
paged-cache unit tests (src/model_runner/server/kv_cache/paged_cache.rs), as data.

Every case runs on one KV head with head_dim 1 and u32 values, as the
reference's tests do: an append at `start` of `count` tokens carries keys
start .. start+count-1 and values 100+start .. 100+start+count-1
(cache_tensor, paged_cache.rs:478-487).  `truncate` keeps the first n tokens
and releases the pages past ceil(n / page_size) (request_state.rs:106-110, :171-178).
Expected values are the ones the tests assert.
Run: python tests/golden/make_kv_append_kats.py
"""
import json
import os


def main():
    cases = []
    # paged_cache.rs:560-587  allocates_pages_for_short_full_and_long_prompts
    for page_size, count, pages in [(16, 15, 1), (16, 16, 1), (16, 17, 2), (2, 3, 2)]:
        cases.append(dict(name=f"allocates_pages_for_short_full_and_long_prompts[{page_size},{count}]",
                          source="paged_cache.rs:560-587", page_size=page_size, ops=[["append", 0, count]],
                          expected_pages=pages, expected_key=list(range(count)),
                          expected_value=list(range(100, 100 + count))))
    # paged_cache.rs:589-610  preserves_values_across_appends
    cases.append(dict(name="preserves_values_across_appends", source="paged_cache.rs:589-610", page_size=2,
                      ops=[["append", 0, 1], ["append", 1, 3], ["append", 4, 2]], expected_pages=3,
                      expected_key=list(range(6)), expected_value=list(range(100, 106))))
    # paged_cache.rs:611-629  truncates_before_reuse
    cases.append(dict(name="truncates_before_reuse", source="paged_cache.rs:611-629", page_size=2,
                      ops=[["append", 0, 6], ["truncate", 3], ["append", 3, 2]], expected_pages=3,
                      expected_key=list(range(5)), expected_value=list(range(100, 105))))
    # paged_cache.rs:640-654  appends_across_a_page_boundary
    cases.append(dict(name="appends_across_a_page_boundary", source="paged_cache.rs:640-654", page_size=16,
                      ops=[["append", 0, 15], ["append", 15, 3]], expected_pages=2,
                      expected_key=list(range(18)), expected_value=list(range(100, 118))))
    # paged_cache.rs:922-1017  adopts_duplicate_pages_across_layers_and_preserves_the_partial_tail:
    # after adopting two canonical read-only prefix pages, the private partial tail stays writable and
    # an append at position 5 lands in it.
    cases.append(dict(name="adopts_duplicate_pages_and_preserves_the_partial_tail", source="paged_cache.rs:922-1017",
                      page_size=2, ops=[["append", 0, 5], ["adopt_prefix_pages", 2], ["append", 5, 1]],
                      expected_pages=3, expected_key=list(range(6)), expected_value=list(range(100, 106))))
    out = dict(source="src/model_runner/server/kv_cache/paged_cache.rs", value_offset=100, cases=cases,
               read_only_message="cannot mutate written physical page {}",
               read_only_source="physical_page_pool.rs:197-201",
               empty_message="cannot append an empty KV-cache tensor", empty_source="kv_cache/utils.rs:33-36")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kv_append_kats.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
