"""Drop-in integrations of the MI355X MSDA operator with third-party libraries.

Each module adapts one library and nothing is re-exported, so importing this
package imports no third-party code (reference ``integrations/__init__.py``).
Import a module directly::

    from deformops_amd.integrations.transformers import patch
"""
