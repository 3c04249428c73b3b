"""Inputs of the front-end golden vectors (shared by make_golden.py and the
tests that read tests/golden/frontend.npz)."""

IPV4 = r"([0-9]{1,3}\.){3}[0-9]{1,3}"
EMAIL = r"[a-z0-9._]{1,32}@[a-z0-9-]{1,24}\.(com|org|net|io)"

PATTERNS = [
    "[01]+", "a+b*", "(ab)+", "-?[0-9]+(\\.[0-9]+)?", "a|bc|12", "[a-c]*", "caf(e|)",
    "aa+", "c", "caf(é|e)", "[^a-c]{2,3}x?", "\\d+\\.\\w*\\s", "(a|b)*abb", ".{0,2}z",
    "[é-ö一-丏]+", "x{3}y{2,}z{0,1}", IPV4, EMAIL,
]

PDA_VOCAB = (["(", ")", "x", "y", "{", "}", "a", "b", ":", "0", "1", ",", "<eos>"], 12)

GRAMMARS = [
    'root ::= "(" root ")" | "x" | "y"',
    'root ::= "{" p ("," p)* "}"\np ::= [a-b] ":" [0-1]',
    'root ::= "x" | "y"',
    'root ::= "yes" | "no"',
    'root ::= field ("," field)*\nfield ::= [a-z]+',
    'root  ::= "[" (val ("," val)*)? "]"\nval   ::= "[" (val ("," val)*)? "]" | [0-9]+',
    'root ::= sign? [0-9]+ frac?\nsign ::= "-"\nfrac ::= "." [0-9]+',
    r'''
root   ::= value
value  ::= object | array | string | number | "true" | "false" | "null"
object ::= "{" [ \t\n]* ( member ( [ \t\n]* "," [ \t\n]* member )* [ \t\n]* )? "}"
member ::= string [ \t\n]* ":" [ \t\n]* value
array  ::= "[" [ \t\n]* ( value ( [ \t\n]* "," [ \t\n]* value )* [ \t\n]* )? "]"
string ::= "\"" ( [^"\\\x00-\x1F] | "\\" ["\\/bfnrt] )* "\""
number ::= "-"? ( "0" | [1-9] [0-9]* ) ( "." [0-9]+ )? ( [eE] [+-]? [0-9]+ )?
''',
]

SCHEMAS = [
    {
        "type": "object",
        "properties": {
            "name": {"type": "string", "maxLength": 24},
            "year": {"type": "integer"},
            "compiled": {"type": "boolean"},
        },
        "required": ["name", "year", "compiled"],
        "additionalProperties": False,
    },
    {
        "type": "object",
        "properties": {"id": {"type": "integer"}, "tags": {"type": "array", "items": {"enum": ["a", "b"]},
                                                          "maxItems": 2}},
        "required": ["id"],
    },
]
