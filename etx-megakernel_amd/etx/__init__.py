"""etx (MI355X build): the batch-small decode megakernel behind the reference's etx.api / etx.operators surface.

Import with the package directory etx-megakernel_amd/ on sys.path.
"""
__all__ = ["api", "operators", "runtime", "models"]
