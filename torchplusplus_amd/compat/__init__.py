"""Stand-ins for the reference's top-level compiled modules.

`import torchplusplus_amd` registers an import hook so that
`import rmsnormFused` (and the other four names) resolve here; adding this
directory to PYTHONPATH has the same effect without the hook.
"""
