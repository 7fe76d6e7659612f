"""Write tests/golden/reference_cases.json: the known answers that the
reference's own hot-path tests assert, transcribed as data (inputs and
expected outputs), with the test file:line each comes from.  Nothing from the
reference is imported or executed; the values are read off the test sources.

Run: python tests/golden/make_reference_cases.py
"""
import json
import os

NEG = -4.0
cases = {
    "source_note": "values transcribed from the reference tests named in each case",
    "greedy_sampler": {
        "source": "runtime/tests/test_sampling.py:40-44 (make_sampler(temp=0) on linspace(-1,1,128) -> 127)",
        "linspace": [-1.0, 1.0, 128],
        "temperature": 0.0,
        "expected_token": 127,
    },
    "greedy_verify_first_mismatch": {
        "source": "runtime/tests/test_runtime.py:1514-1532",
        "draft_tokens": [2, 4],
        "draft_logprobs": [[0.0] * 5, [0.0] * 5],
        "target": [[NEG, NEG, 0.0, NEG, NEG], [NEG, NEG, NEG, 0.0, NEG], [NEG, 0.0, NEG, NEG, NEG]],
        "temperature": 0.0,
        "expected_accepted": 1,
        "expected_token": 3,
    },
    "sampling_verify_identical": {
        "source": "runtime/tests/test_runtime.py:1534-1542",
        "draft_tokens": [1],
        "draft_logprobs": [["-inf", 0.0, "-inf"]],
        "target": [["-inf", 0.0, "-inf"], ["-inf", 0.0, "-inf"]],
        "temperature": 1.0,
        "expected_accepted": 1,
        "expected_token": 1,
    },
    "mtp_disjoint_supports": {
        "source": "runtime/tests/test_qwen.py:420-442 (target supports {0}, draft supports {1}: "
                  "round (1 proposed, 0 accepted), every emitted token is 0)",
        "vocab": 32,
        "target_support": [0],
        "draft_support": [1],
        "temperature": 1.0,
        "expected_accepted": 0,
        "expected_token": 0,
    },
    "mtp_identical_supports": {
        "source": "runtime/tests/test_qwen.py:387-418 (supports {0,1} on both sides, T=0.7, top_p=0.8, "
                  "top_k=2: the single draft is accepted)",
        "vocab": 32,
        "support": [0, 1],
        "temperature": 0.7,
        "top_p": 0.8,
        "top_k": 2,
        "expected_accepted": 1,
    },
    "greedy_mtp_chain": {
        "source": "runtime/tests/test_qwen.py:360-385 (target predicts token+1 mod 32 with +-1000 logits; "
                  "prompt [1,2], 7 tokens -> [3,4,5,6,7,8,9], five drafts all accepted)",
        "vocab": 32,
        "expected_tokens": [3, 4, 5, 6, 7, 8, 9],
        "expected_round": [5, 5],
    },
    "greedy_mtp_partial": {
        "source": "runtime/tests/test_qwen.py:468-490 (draft mispredicts after input 5: round (3, 2), "
                  "tokens [3,4,5,6,7])",
        "vocab": 32,
        "expected_tokens": [3, 4, 5, 6, 7],
        "expected_round": [3, 2],
    },
    "qwen_chat_defaults": {
        "source": "runtime/tests/test_advanced_defaults.py:18-24 (adaptive chat: T 0.7, top_p 0.8, top_k 20, "
                  "presence 1.5; thinking: T 1.0, top_p 0.95, top_k 20, presence 0)",
        "chat": {"temperature": 0.7, "top_p": 0.8, "top_k": 20, "presence_penalty": 1.5},
        "thinking": {"temperature": 1.0, "top_p": 0.95, "top_k": 20, "presence_penalty": 0.0},
    },
    "sampler_profiles": {
        "source": "runtime/tests/test_sampling.py:23-24",
        "profiles": [
            {"temp": 1.0},
            {"temp": 1.0, "top_p": 0.95, "top_k": 20},
            {"temp": 0.7, "top_p": 0.8, "top_k": 20, "min_p": 0.05},
        ],
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_cases.json")
    with open(out, "w") as f:
        json.dump(cases, f, indent=1)
    print("wrote", out)
