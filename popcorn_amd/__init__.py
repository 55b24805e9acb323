"""popcorn_amd: an MI355X (gfx950) kernel backend for Popcorn's transformer-block ops.

`popcorn_amd.impls` holds the reference-signature implementations,
`popcorn_amd.backend.register(popcorn)` registers them with a Popcorn
dispatcher, and `popcorn_amd.compat` is a self-contained counterpart of
Popcorn's registration / validation / selection surface for environments
without Popcorn itself.
"""

__version__ = "0.1.0"
