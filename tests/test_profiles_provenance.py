"""Every measurement summary under profiles/ that names the kernel sources it was measured on
names the sources in the tree, so a change to a kernel's code without fresh measurements fails
here. A summary names its build as a backticked 16-hex-digit digest (text) or a ``build`` /
``source_digest`` value (JSON); summaries that name no build (older counter studies) are not
checked. No device is needed."""

from __future__ import annotations

import json
import re
from pathlib import Path

import bench

PROFILES = Path(__file__).resolve().parent.parent / "profiles"
_TEXT_DIGEST = re.compile(r"`([0-9a-f]{16})`")


def _json_digests(node: object) -> list[str]:
    if isinstance(node, dict):
        found = [v for k, v in node.items() if k in ("build", "source_digest") and isinstance(v, str)]
        return found + [d for v in node.values() for d in _json_digests(v)]
    if isinstance(node, list):
        return [d for v in node for d in _json_digests(v)]
    return []


def named_builds(path: Path) -> list[str]:
    text = path.read_text()
    if path.suffix == ".json":
        return _json_digests(json.loads(text))
    return _TEXT_DIGEST.findall(text)


def test_digest_reader_finds_both_forms(tmp_path: Path) -> None:
    md = tmp_path / "a.md"
    md.write_text("Kernel sources `0123456789abcdef`; kernel `decode_kernel<1>` (`fedcba9876543210`).")
    js = tmp_path / "a.json"
    js.write_text(json.dumps({"runs": [{"build": "00112233445566aa"}], "source_digest": "ffeeddccbbaa9988"}))
    assert named_builds(md) == ["0123456789abcdef", "fedcba9876543210"]
    assert sorted(named_builds(js)) == ["00112233445566aa", "ffeeddccbbaa9988"]


def test_stamped_profiles_name_the_current_kernel_sources() -> None:
    current = bench.source_digest()
    stamped = {p.name: named_builds(p) for p in sorted(PROFILES.iterdir()) if p.suffix in (".md", ".txt", ".json")}
    named = {name: builds for name, builds in stamped.items() if builds}
    assert len(named) >= 5, f"expected the stamped summaries, found {sorted(named)}"
    stale = {name: builds for name, builds in named.items() if any(b != current for b in builds)}
    assert not stale, f"kernel sources are {current}; summaries measured on other sources: {stale}"
