"""The harness around the backends: plugin contract, catalog, drivers, checks and reports."""
