"""Erases the TypeScript types of runntime_amd/napi/hipExecutor.ts so the
image's Node 12 can run it (Node >= 22, the reference's runtime, strips
them itself).

It handles the erasable subset that file is written in, and no more:
`import type` lines, `interface` blocks, `implements` clauses, `readonly`
modifiers, `as T` casts, postfix `!`, and annotations written `name: Type`
/ `name?: Type` / `): Type` with no space before the colon (the file's
ternaries put spaces around their colon and it has no `key: value`
object literals). The test that uses it checks the result parses and
behaves, so a construct it misses fails loudly."""
import re
import sys

_NAME = r"[A-Za-z_][\w.]*"
_TYPE1 = rf"(?:readonly\s+)?{_NAME}(?:<[^<>;{{}}]*(?:<[^<>]*>)?[^<>;{{}}]*>)?(?:\[\])*"
_TYPE = rf"{_TYPE1}(?:\s*\|\s*{_TYPE1})*"


def strip(ts: str) -> str:
    out, lines, i = [], ts.split("\n"), 0
    while i < len(lines):
        line = lines[i]
        if re.match(r"\s*import type\b", line):
            i += 1
            continue
        if re.match(r"\s*(export\s+)?interface\s", line):
            depth = line.count("{") - line.count("}")
            i += 1
            while depth > 0 and i < len(lines):
                depth += lines[i].count("{") - lines[i].count("}")
                i += 1
            continue
        out.append(line)
        i += 1
    js = "\n".join(out)
    js = re.sub(r"\s+implements\s+[\w\s,]+(?=\{)", " ", js)
    js = re.sub(r"\bas\s+unknown\s+as\s+" + _NAME, "", js)
    js = re.sub(r"\s+as\s+[A-Z]\w*(?:\[\])*(?=[\s;,)\]])", "", js)
    js = re.sub(r"\breadonly\s+(?=#|\w+\s*[:=;])", "", js)
    # annotations: an identifier or ')' directly followed by ':' / '?:'
    js = re.sub(rf"(?<=[\w)])\??:[ ]*{_TYPE}(?=\s*(?:[,)=;{{]|=>|$))", "", js, flags=re.M)
    # postfix non-null assertions
    js = re.sub(r"(?<=[\w\])])!(?!=)", "", js)
    return js


if __name__ == "__main__":
    sys.stdout.write(strip(open(sys.argv[1]).read()))
